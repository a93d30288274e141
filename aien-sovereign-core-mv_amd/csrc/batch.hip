// Batched serving decode for gfx950 (omega_gpu_batch_decode_*): one greedy decode step of up to
// 32 sequences of the Qwen3-30B-A3B FP8 model over the caller's paged KV pool (the aien-kv-cache
// page layout, read and written in place), captured as one hipGraph per batch size.
//
// Reference semantics: the engine step for one token (crates/aien-inference-abi/src/
// qwen3_moe_omega.rs:4096-4345) applied to each sequence — input RMSNorm, q|k|v FP8 projection,
// per-head q/k RMSNorm and RoPE (qwen3_coder.rs:306-320, tensor.rs:150-190), the token's K/V
// appended as bf16 (aien-kv-cache write_token_kv), attention over the sequence's pages
// (tensor.rs:193-250), o projection into the residual, the MoE block (router, top-8, gate|up,
// SwiGLU, down, slot-order combine) into the residual; then the final norm, the bf16 lm_head and
// the lowest-index argmax (tensor.rs:299-318). The sequences share every weight read: the
// projections are FP8 matrix-core GEMMs over the batch, the experts are grouped by expert
// (moe.hip), the attention is the ragged paged kernel (attn.hip), the lm_head a bf16 matrix-core
// GEMM with the argmax folded in. Only the MoE planner exchanges data between the workgroups of
// one launch (its rankings, then the grouping).
//
// Per layer: rows (the previous layer's MoE combine into the residual, norm + split) | q|k|v GEMM
// (k-slice partials) | q/k norm, RoPE, K/V append | paged attention items | combine + split |
// o GEMM (k-slice partials) | MoE block (5 launches, its first adds the o partials into the
// residual; its combine is left to the next rows launch). Then final norm (with the last
// layer's combine) | lm_head + argmax.
#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdio>
#include <map>
#include <vector>

#include "device.hpp"
#include "kernels.hpp"
#include "mfma.hpp"
#include "route.hpp"
#include "runtime.hpp"

namespace omega {
RouterArgs router_args(const OmegaGpuRouter *r, uint32_t layer, const float *x, float eps,
                       int norm_topk, float out_scale);
uint32_t router_layers(const OmegaGpuRouter *r);
uint32_t router_rows(const OmegaGpuRouter *r);
KvGeom geom_of(const OmegaGpuKvLayout &l);
void rope_table(double theta, uint32_t positions, float *cos_out, float *sin_out);

constexpr uint32_t kBdH = 2048, kBdQkv = 5120, kBdAttn = 4096;
constexpr uint32_t kBdMaxSeqs = 32;
static_assert(kBdMaxSeqs <= kItemMaxSeqs, "the attention plan covers every sequence");

// the device words the host writes before every step (and the argmax slots it reads back)
struct BdIo {
    uint32_t tok[kBdMaxSeqs];
    uint32_t pos[kBdMaxSeqs];           // the token's position: its KV slot; context = pos + 1
    ItemPlan plan;                      // the step's attention work items
    uint32_t moe_late;                  // MoE planner waits that ran out this step
    uint32_t plan_epoch;                // the step's MoE planner epoch base (layer l: * 64 + l)
    unsigned long long argmax[kBdMaxSeqs][kArgmaxSlots];
};
static_assert(offsetof(BdIo, argmax) % 8 == 0, "argmax slots 8-byte aligned");
static_assert(offsetof(BdIo, argmax) == offsetof(BdIo, moe_late) + 8, "one copy back: moe_late, argmax");
// the step's results copied back in one transfer: the planner's count, then seqs argmax rows
constexpr size_t bd_back_bytes(uint32_t seqs) {
    return 8 + sizeof(unsigned long long) * kArgmaxSlots * seqs;
}

struct BdArgs {
    uint32_t T = 0;
    BdIo *io = nullptr;
    const uint16_t *embed = nullptr;  // layer 0: x = embedding row of the token
    uint32_t vocab = 0;
    const float *norm_w = nullptr;    // rows: the layer's input norm; final: the final norm
    const float *q_norm = nullptr, *k_norm = nullptr;
    float eps = 1e-6f;
    const float *rope_cos = nullptr, *rope_sin = nullptr;  // [max_pos][64]
    uint8_t *pool = nullptr;
    KvGeom g{};
    uint32_t layer = 0;
    const int32_t *tables = nullptr;  // [T][max_blocks]
    uint32_t max_blocks = 0;
    float *x = nullptr;               // [T][2048] residual rows
    uint8_t *xq = nullptr;            // [T][16][4][128] split input rows of q|k|v
    float *xs = nullptr;              // [T][16][4]
    const float *qkv_part = nullptr;  // [8][T][5120]
    float *q = nullptr;               // [T][32][128]
    float *hidden = nullptr;          // [T][2048] final-normed rows
    uint16_t *hid_hi = nullptr, *hid_lo = nullptr;  // their bf16 hi / lo halves
    // the previous layer's MoE combine, done by this launch (null: none pending)
    const float *moe_dp = nullptr;         // [T * 8][2048] down rows
    const uint32_t *moe_row = nullptr;     // [T * 8] grouped row of pair t * 8 + s
    const float *moe_w = nullptr;          // [T * 8] slot weights
    int moe_mutant = 0;                    // 6: slot 7 dropped
};

// x[t][8 tid .. +8] += the token's MoE row: its slots' down rows weighted, summed in slot order
// from zero (the arithmetic of the MoE block's combine), written back as the residual row
__device__ __forceinline__ void bd_moe_combine(const BdArgs &a, uint32_t t, uint32_t tid, float *xr, float (&v)[8]) {
    float moe[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kTopK; ++s) {
        const uint32_t row = as_const_u32(a.moe_row)[t * kTopK + s];
        const float w = (a.moe_mutant == 6 && s == kTopK - 1) ? 0.f : __uint_as_float(as_const_u32(a.moe_w)[t * kTopK + s]);
        const float *y = a.moe_dp + (size_t)row * kBdH + 8 * tid;
        const f32x4 y0 = *as_global_f32x4(y), y1 = *as_global_f32x4(y + 4);
        const float yv[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) moe[i] += w * yv[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = v[i] + moe[i];
    *reinterpret_cast<f32x4 *>(xr) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4 *>(xr + 4) = f32x4{v[4], v[5], v[6], v[7]};
}

// ------------------------------------------------------------------ rows: (embedding) + RMSNorm + split
__global__ __launch_bounds__(256) void k_bd_rows(const BdArgs a) {
    __shared__ double red[4];
    const uint32_t t = blockIdx.x, tid = threadIdx.x, lane = lane_id(), wid = tid >> 6;
    float v[8];
    float *xr = a.x + (size_t)t * kBdH + 8 * tid;
    if (a.embed) {
        const uint32_t tok = a.io->tok[t] % a.vocab;
        const u32x4 e = *as_global(a.embed + (size_t)tok * kBdH + 8 * tid);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[2 * j] = bf16_lo(e[j]);
            v[2 * j + 1] = bf16_hi(e[j]);
        }
        *reinterpret_cast<f32x4 *>(xr) = f32x4{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f32x4 *>(xr + 4) = f32x4{v[4], v[5], v[6], v[7]};
    } else {
        const f32x4 h0 = *as_global_f32x4(xr), h1 = *as_global_f32x4(xr + 4);
        v[0] = h0.x; v[1] = h0.y; v[2] = h0.z; v[3] = h0.w;
        v[4] = h1.x; v[5] = h1.y; v[6] = h1.z; v[7] = h1.w;
        if (a.moe_dp) bd_moe_combine(a, t, tid, xr, v);
    }
    const f32x4 w0 = *as_global_f32x4(a.norm_w + 8 * tid), w1 = *as_global_f32x4(a.norm_w + 8 * tid + 4);
    const float nw[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += (double)v[i] * (double)v[i];
    ss = wave_sum_f64(ss);
    if (lane == 0) red[wid] = ss;
    __syncthreads();
    const float scale = rms_scale((red[0] + red[1]) + (red[2] + red[3]), kBdH, a.eps);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = v[i] * scale * nw[i];
    u32x2 q[kTerms];
    float s[kTerms];
    split8(v, q, s, false);
    store_split(a.xq, a.xs, t, kBdH / 128, tid >> 4, tid & 15, q, s);
}

// ------------------------------------------------------------------ dense FP8 GEMM (the batch's rows)
// A workgroup = (4 tiles of 32 weight rows, k-slice of 2 blocks), all T <= 16 MT rows. The
// slice's activation terms of every row (16 MT rows x 1 KiB) are staged once per workgroup in
// LDS, so each of the four wavefronts reads them there instead of from L2 (the terms are four
// times the weights' bytes per wavefront); each wavefront's tile weights (8 KiB from the tiled
// twin, 1 KiB contiguous per load instruction) go out first, then the products and the partial
// sums of the k-slice. One tile per wavefront puts the whole weight stream in flight at once
// (q|k|v: 160 tiles x 8 slices = 1280 wavefronts). Scales come through scalar loads and every
// store is unconditional (rows past T write the sink), so no wait merges over a branch.
struct DenseArgs {
    const uint8_t *wt = nullptr;  // tiled twin of a [1][n][k] FP8 tensor
    const float *s = nullptr;     // [n/128][k/128]
    uint32_t n = 0, k = 0;
    const uint8_t *xq = nullptr;  // [T][k/128][4][128]
    const float *xs = nullptr;    // [T][k/128][4]
    uint32_t T = 0;
    float *part = nullptr;        // [k/256][T][n]
    float *sink = nullptr;        // [64]: where the lanes of rows past T store
};

// k-blocks per slice: q|k|v (k = 2048) 2, o_proj (k = 4096) 4, so both write 8 k-slices
constexpr uint32_t dense_kbw(uint32_t k) { return k >= 4096 ? 4 : 2; }
constexpr uint32_t kDenseSlices = 8;

template <int MT, int KBW>
__global__ __launch_bounds__(256) void k_dense_gemm(const DenseArgs a) {
    constexpr uint32_t kDenseRowBytes = KBW * kTerms * 128;  // a row's terms of one slice
    constexpr uint32_t kDensePitch = kDenseRowBytes + 16;     // LDS row pitch (rows 4 banks apart)
    __shared__ __align__(16) uint8_t bl[MT * 16 * kDensePitch];
    const uint32_t lane = lane_id(), g = lane >> 4, n = lane & 15, wid = threadIdx.x >> 6;
    const uint32_t KB = a.k / 128, splits = KB / KBW;
    const uint32_t split = blockIdx.x % splits, tile = (blockIdx.x / splits) * 4 + wid;
    const uint32_t kb0 = split * KBW;
    MoeTileA<KBW> A;
    A.load(a.wt + ((size_t)(2 * tile) * KB + kb0) * 2048, a.wt + ((size_t)(2 * tile + 1) * KB + kb0) * 2048, lane);
    // the slice's terms of all 16 MT rows (rows past T repeat row T - 1): 1 KiB contiguous per row
    constexpr uint32_t kChunks = MT * 16 * kDenseRowBytes / 16;
    u32x4 st[kChunks / 256];
#pragma unroll
    for (uint32_t c = 0; c < kChunks / 256; ++c) {
        const uint32_t ch = threadIdx.x + 256 * c, row = ch / (kDenseRowBytes / 16), off = 16 * (ch % (kDenseRowBytes / 16));
        const uint32_t tok = min(row, a.T - 1);
        st[c] = *as_global(a.xq + ((size_t)tok * KB + kb0) * kTerms * 128 + off);
    }
    // the terms' scales of the lane's rows
    int sbe[MT][KBW][kTerms];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const uint32_t tok = min(16 * m + n, a.T - 1);
        const float *sr = a.xs + ((size_t)tok * KB + kb0) * 4;
#pragma unroll
        for (int j = 0; j < KBW; ++j) {
            const f32x4 v = *as_global_f32x4(sr + 4 * j);
            sbe[m][j][0] = e8m0_of(v.x);
            sbe[m][j][1] = e8m0_of(v.y);
            sbe[m][j][2] = e8m0_of(v.z);
            sbe[m][j][3] = e8m0_of(v.w);
        }
    }
#pragma unroll
    for (uint32_t c = 0; c < kChunks / 256; ++c) {
        const uint32_t ch = threadIdx.x + 256 * c, row = ch / (kDenseRowBytes / 16), off = 16 * (ch % (kDenseRowBytes / 16));
        *reinterpret_cast<u32x4 *>(bl + row * kDensePitch + off) = st[c];
    }
    __syncthreads();  // n is a multiple of 128, so every wavefront has a tile
    const cu32 *ws = as_const_u32(a.s + (size_t)((32 * tile) >> 7) * KB + kb0);
    float *part = a.part + (size_t)split * a.T * a.n;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        // lane (g, n): row 16 m + n, bytes 16 g and 64 + 16 g of each 128-byte term
        const uint8_t *br = bl + (16 * m + n) * kDensePitch + 16 * g;
        i32x8 B[KBW][kTerms];
#pragma unroll
        for (int j = 0; j < KBW; ++j)
#pragma unroll
            for (uint32_t t = 0; t < kTerms; ++t) {
                const u32x4 lo = *reinterpret_cast<const u32x4 *>(br + (j * kTerms + t) * 128);
                const u32x4 hi = *reinterpret_cast<const u32x4 *>(br + (j * kTerms + t) * 128 + 64);
                B[j][t] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
        f32x4 tot[2];
        tot[0] = tot[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < KBW; ++j) {
            const float w = __uint_as_float(ws[j]);
            f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (uint32_t t = 0; t < kTerms; ++t) {
                c0 = mfma_fp8_sb(A.A[0][j], B[j][t], c0, sbe[m][j][t]);
                c1 = mfma_fp8_sb(A.A[1][j], B[j][t], c1, sbe[m][j][t]);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                tot[0][q] = fmaf(c0[q], w, tot[0][q]);
                tot[1][q] = fmaf(c1[q], w, tot[1][q]);
            }
        }
        const uint32_t tok = 16 * m + n;
        float *y = (tok < a.T ? part + (size_t)tok * a.n + 32 * tile : a.sink) + 4 * g;
        *reinterpret_cast<f32x4 *>(y) = tot[0];
        *reinterpret_cast<f32x4 *>(y + 16) = tot[1];
    }
}

hipError_t launch_dense_gemm(const DenseArgs &a, hipStream_t st) {
    // workgroups of 4 tiles of 32 rows, one per (tile group, k-slice)
    const uint32_t kbw = dense_kbw(a.k);
    if (a.n % 128 || a.k != kDenseSlices * 128 * kbw || a.T == 0 || a.T > 32) return hipErrorInvalidValue;
    const uint32_t wgs = kDenseSlices * (a.n / 128);
    if (kbw == 2) {
        if (a.T <= 16) OMEGA_LAUNCH((k_dense_gemm<1, 2>), dim3(wgs), dim3(256), 0, st, a);
        else OMEGA_LAUNCH((k_dense_gemm<2, 2>), dim3(wgs), dim3(256), 0, st, a);
    } else {
        if (a.T <= 16) OMEGA_LAUNCH((k_dense_gemm<1, 4>), dim3(wgs), dim3(256), 0, st, a);
        else OMEGA_LAUNCH((k_dense_gemm<2, 4>), dim3(wgs), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ q|k|v: norms, RoPE, K/V append
// one wavefront per (sequence, kv head): the 8 q heads, k and v summed over the GEMM's 8 k-slices,
// per-head RMSNorm (f64 sums of squares) and RoPE at the sequence's position; q stored for the
// attention, K and V rounded to bf16 and written into the sequence's page slot.
__global__ __launch_bounds__(64) void k_bd_qkv(const BdArgs a) {
    const uint32_t t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const uint32_t pos = a.io->pos[t];
    const size_t slice = (size_t)a.T * kBdQkv;
    const float *base = a.qkv_part + (size_t)t * kBdQkv;
    auto sum8 = [&](uint32_t col) {
        float v = 0.f;
#pragma unroll
        for (uint32_t k = 0; k < 8; ++k) v += *as_global_f32(base + k * slice + col);
        return v;
    };
    float q0[8], q1[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        q0[r] = sum8((h * 8 + r) * 128 + lane);
        q1[r] = sum8((h * 8 + r) * 128 + 64 + lane);
    }
    float k0 = sum8(kBdAttn + h * 128 + lane), k1 = sum8(kBdAttn + h * 128 + 64 + lane);
    const float v0 = sum8(kBdAttn + 512 + h * 128 + lane), v1 = sum8(kBdAttn + 512 + h * 128 + 64 + lane);
    const float qw0 = *as_global_f32(a.q_norm + lane), qw1 = *as_global_f32(a.q_norm + 64 + lane);
    const float kw0 = *as_global_f32(a.k_norm + lane), kw1 = *as_global_f32(a.k_norm + 64 + lane);
    const float rc = *as_global_f32(a.rope_cos + (size_t)pos * 64 + lane);
    const float rs = *as_global_f32(a.rope_sin + (size_t)pos * 64 + lane);
    double ss[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) ss[r] = (double)q0[r] * (double)q0[r] + (double)q1[r] * (double)q1[r];
    const float scale_l = rms_scale(head_sums8(ss, lane), 128, a.eps);  // lane l: head l / 8
    float *qo = a.q + ((size_t)t * 32 + h * 8) * 128;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        head_scale_rope(q0[r], q1[r], readlane_f32(scale_l, 8 * r), qw0, qw1, rc, rs, true);
        qo[r * 128 + lane] = q0[r];
        qo[r * 128 + 64 + lane] = q1[r];
    }
    const float kscale = rms_scale(wave_sum_f64((double)k0 * (double)k0 + (double)k1 * (double)k1), 128, a.eps);
    head_scale_rope(k0, k1, kscale, kw0, kw1, rc, rs, true);
    const uint32_t blk = (uint32_t)a.tables[(size_t)t * a.max_blocks + pos / 16];
    uint16_t *krow = reinterpret_cast<uint16_t *>(a.pool + kv_row_offset(a.g, blk, a.layer, 0, pos % 16, h));
    uint16_t *vrow = reinterpret_cast<uint16_t *>(a.pool + kv_row_offset(a.g, blk, a.layer, 1, pos % 16, h));
    krow[lane] = bf16_rne(k0);
    krow[lane + 64] = bf16_rne(k1);
    vrow[lane] = bf16_rne(v0);
    vrow[lane + 64] = bf16_rne(v1);
}

// ------------------------------------------------------------------ final norm -> bf16 hi / lo
__global__ __launch_bounds__(256) void k_bd_final(const BdArgs a) {
    __shared__ double red[4];
    const uint32_t t = blockIdx.x, tid = threadIdx.x, lane = lane_id(), wid = tid >> 6;
    float *xr = a.x + (size_t)t * kBdH + 8 * tid;
    const f32x4 h0 = *as_global_f32x4(xr), h1 = *as_global_f32x4(xr + 4);
    float v[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
    if (a.moe_dp) bd_moe_combine(a, t, tid, xr, v);
    const f32x4 w0 = *as_global_f32x4(a.norm_w + 8 * tid), w1 = *as_global_f32x4(a.norm_w + 8 * tid + 4);
    const float nw[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += (double)v[i] * (double)v[i];
    ss = wave_sum_f64(ss);
    if (lane == 0) red[wid] = ss;
    __syncthreads();
    const float scale = rms_scale((red[0] + red[1]) + (red[2] + red[3]), kBdH, a.eps);
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = v[i] * scale * nw[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        hi[j] = (uint32_t)bf16_split_hi(v[2 * j]) | ((uint32_t)bf16_split_hi(v[2 * j + 1]) << 16);
        lo[j] = (uint32_t)bf16_split_lo(v[2 * j]) | ((uint32_t)bf16_split_lo(v[2 * j + 1]) << 16);
    }
    float *ho = a.hidden + (size_t)t * kBdH + 8 * tid;
    *reinterpret_cast<f32x4 *>(ho) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4 *>(ho + 4) = f32x4{v[4], v[5], v[6], v[7]};
    *reinterpret_cast<u32x4 *>(a.hid_hi + (size_t)t * kBdH + 8 * tid) = u32x4{hi[0], hi[1], hi[2], hi[3]};
    *reinterpret_cast<u32x4 *>(a.hid_lo + (size_t)t * kBdH + 8 * tid) = u32x4{lo[0], lo[1], lo[2], lo[3]};
}

// ------------------------------------------------------------------ lm_head (bf16 matrix cores) + argmax
// A wavefront = 64 vocabulary rows (4 tiles of 16) x every row of the batch: per 32-column block
// the 4 tiles' operands from the tiled twin (1 KiB contiguous each) and the rows' hidden bf16 hi
// and lo halves (products with the bf16 weights exact in f32), one block ahead in flight. Each
// row's best (value, lowest index) key goes to one of the row's argmax slots by atomicMax.
struct LmArgs {
    const uint16_t *wt = nullptr;  // tiled twin [n][k]
    uint32_t n = 0, k = 0;
    const uint16_t *hi = nullptr, *lo = nullptr;  // [T][k]
    uint32_t T = 0;
    float *logits = nullptr;       // [T][n] or null
    unsigned long long *argmax = nullptr;  // [kBdMaxSeqs][kArgmaxSlots]
};

template <int MT>
__global__ __launch_bounds__(256) void k_bd_lm(const LmArgs a) {
    const uint32_t lane = lane_id(), g = lane >> 4, n = lane & 15;
    const uint32_t w = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    const uint32_t rts = a.n / 16, rt0 = 4 * w;
    if (rt0 >= rts) return;
    const uint32_t R = min(4u, rts - rt0), KB = a.k / 32;
    auto ldA = [&](uint32_t r, uint32_t kb) {
        const uint16_t *b = a.wt + ((size_t)(rt0 + min(r, R - 1)) * KB + kb) * 512 + 8 * lane;
        return as_bf16x8(__builtin_nontemporal_load(as_global(b)));
    };
    auto ldB = [&](const uint16_t *src, uint32_t m, uint32_t kb) {
        const uint32_t tok = min(16 * m + n, a.T - 1);
        return as_bf16x8(*as_global(src + (size_t)tok * a.k + 32 * kb + 8 * g));
    };
    f32x4 acc[4][MT];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = f32x4{0.f, 0.f, 0.f, 0.f};
    bf16x8 A[4], Bh[MT], Bl[MT];
#pragma unroll
    for (int r = 0; r < 4; ++r) A[r] = ldA(r, 0);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        Bh[m] = ldB(a.hi, m, 0);
        Bl[m] = ldB(a.lo, m, 0);
    }
#pragma unroll 1
    for (uint32_t kb = 0; kb < KB; ++kb) {
        const uint32_t kn = kb + 1 < KB ? kb + 1 : kb;
        bf16x8 An[4], Bhn[MT], Bln[MT];
#pragma unroll
        for (int r = 0; r < 4; ++r) An[r] = ldA(r, kn);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            Bhn[m] = ldB(a.hi, m, kn);
            Bln[m] = ldB(a.lo, m, kn);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                acc[r][m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[r], Bh[m], acc[r][m], 0, 0, 0);
                acc[r][m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[r], Bl[m], acc[r][m], 0, 0, 0);
            }
#pragma unroll
        for (int r = 0; r < 4; ++r) A[r] = An[r];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            Bh[m] = Bhn[m];
            Bl[m] = Bln[m];
        }
    }
    // lane (g, n): rows (rt0 + r) * 16 + 4 g + i of batch row 16 m + n
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const uint32_t tok = 16 * m + n;
        unsigned long long best = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if ((uint32_t)r >= R) break;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t row = (rt0 + r) * 16 + 4 * g + i;
                const float v = acc[r][m][i];
                if (a.logits && tok < a.T) a.logits[(size_t)tok * a.n + row] = v;
                const unsigned long long key = argmax_key(v, row);
                best = key > best ? key : best;
            }
        }
        // the 4 lane groups of a column hold 16 rows each: the maximum over them
#pragma unroll
        for (int sh = 16; sh <= 32; sh <<= 1) {
            const uint32_t lo32 = (uint32_t)best, hi32 = (uint32_t)(best >> 32);
            const uint32_t olo = (uint32_t)__shfl_xor((int)lo32, sh, 64), ohi = (uint32_t)__shfl_xor((int)hi32, sh, 64);
            const unsigned long long o = ((unsigned long long)ohi << 32) | olo;
            best = o > best ? o : best;
        }
        if (g == 0 && tok < a.T && best) atomicMax(&a.argmax[(size_t)tok * kArgmaxSlots + w % kArgmaxSlots], best);
    }
}

hipError_t launch_bd_lm(const LmArgs &a, hipStream_t st) {
    const uint32_t waves = (a.n / 16 + 3) / 4;
    if (a.T <= 16) OMEGA_LAUNCH(k_bd_lm<1>, dim3((waves + 3) / 4), dim3(256), 0, st, a);
    else OMEGA_LAUNCH(k_bd_lm<2>, dim3((waves + 3) / 4), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace omega

using namespace omega;

namespace {
struct BdLayer {
    OmegaGpuFp8Tensor *qkv = nullptr, *o = nullptr, *gu = nullptr, *dn = nullptr;
    float *in_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;  // device
};
}  // namespace

struct OmegaGpuBatchDecode {
    OmegaGpuBatchDecodeConfig cfg{};
    OmegaGpuRouter *router = nullptr;
    OmegaGpuBf16Tensor *lm = nullptr, *embed = nullptr;
    KvGeom g{};
    std::vector<BdLayer> layers;
    float *final_norm = nullptr;
    bool final_set = false, tables_set = false;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    // workspace
    float *x = nullptr, *qkv_part = nullptr, *q = nullptr, *apart = nullptr, *o_part = nullptr;
    float *sink = nullptr;  // the dense GEMMs' stores of rows past the batch
    float *hidden = nullptr, *logits = nullptr;
    uint8_t *xq = nullptr, *oq = nullptr;
    float *xs = nullptr, *os = nullptr;
    uint16_t *hid_hi = nullptr, *hid_lo = nullptr;
    int32_t *tables = nullptr;
    void *moe = nullptr;
    uint32_t *route_ids = nullptr;  // [layers][max_seqs][8]
    float *route_w = nullptr;
    BdIo *io = nullptr, *pin = nullptr;
    std::vector<uint32_t> table_pages;  // per sequence: the leading table entries that name a page
    bool keep_logits = false;
    bool eager = false;  // launch the kernels directly (profilers that cannot follow graph capture)
    std::map<uint32_t, hipGraphExec_t> exec;  // key: seqs | keep_logits << 8 | MoE mutant << 9
    std::vector<hipGraph_t> graphs;
};

namespace {

int bd_enqueue(OmegaGpuBatchDecode *b, uint32_t T, hipStream_t st) {
    const OmegaGpuBatchDecodeConfig &c = b->cfg;
    BdArgs a;
    a.T = T;
    a.io = b->io;
    a.vocab = c.vocab;
    a.eps = c.eps;
    a.rope_cos = b->rope_cos;
    a.rope_sin = b->rope_sin;
    a.pool = static_cast<uint8_t *>(c.pool);
    a.g = b->g;
    a.tables = b->tables;
    a.max_blocks = c.max_blocks_per_seq;
    a.x = b->x;
    a.xq = b->xq;
    a.xs = b->xs;
    a.qkv_part = b->qkv_part;
    a.q = b->q;
    a.hidden = b->hidden;
    a.hid_hi = b->hid_hi;
    a.hid_lo = b->hid_lo;
    for (uint32_t l = 0; l < c.layers; ++l) {
        const BdLayer &L = b->layers[l];
        a.layer = l;
        a.embed = l == 0 ? b->embed->w : nullptr;
        a.norm_w = L.in_norm;
        a.q_norm = L.q_norm;
        a.k_norm = L.k_norm;
        OMEGA_LAUNCH(k_bd_rows, dim3(T), dim3(256), 0, st, a);
        DenseArgs dq;
        dq.wt = L.qkv->wt;
        dq.s = L.qkv->s;
        dq.n = kBdQkv;
        dq.k = kBdH;
        dq.xq = b->xq;
        dq.xs = b->xs;
        dq.T = T;
        dq.part = b->qkv_part;
        dq.sink = b->sink;
        OMEGA_HIP(F_SESSION, launch_dense_gemm(dq, st));
        OMEGA_LAUNCH(k_bd_qkv, dim3(T, 4), dim3(64), 0, st, a);
        PagedItemsArgs pa;
        pa.q = b->q;
        pa.pool = static_cast<const uint8_t *>(c.pool);
        pa.g = b->g;
        pa.layer = l;
        pa.tables = b->tables;
        pa.max_blocks = c.max_blocks_per_seq;
        pa.pos = b->io->pos;
        pa.run_off = b->io->plan.run_off;
        pa.items = &b->io->plan.items[0][0];
        pa.part = b->apart;
        OMEGA_HIP(F_SESSION, launch_paged_items(pa, kItemRuns, st));
        CombineItemsArgs ca;
        ca.part = b->apart;
        ca.item_off = b->io->plan.item_off;
        ca.oq = b->oq;
        ca.os = b->os;
        OMEGA_HIP(F_SESSION, launch_attn_combine_items(ca, T, st));
        DenseArgs dO;
        dO.wt = L.o->wt;
        dO.s = L.o->s;
        dO.n = kBdH;
        dO.k = kBdAttn;
        dO.xq = b->oq;
        dO.xs = b->os;
        dO.T = T;
        dO.part = b->o_part;
        dO.sink = b->sink;
        OMEGA_HIP(F_SESSION, launch_dense_gemm(dO, st));
        MoeArgs m;
        moe_work_carve(m, b->moe, T);
        RouterArgs ra = router_args(b->router, l, nullptr, c.eps, c.norm_topk, 1.0f);
        m.gate = ra.gate;
        m.norm_w = ra.norm_w;
        m.eps = c.eps;
        m.norm_topk = c.norm_topk;
        m.tokens = T;
        m.gu_wt = L.gu->wt;
        m.gu_s = L.gu->s;
        m.dn_wt = L.dn->wt;
        m.dn_s = L.dn->s;
        m.gu_w = L.gu->w;
        m.dn_w = L.dn->w;
        m.h = b->x;
        m.opart = b->o_part;
        m.oslices = kDenseSlices;
        m.hout = b->x;
        m.resid = b->x;
        m.out = b->x;
        m.ids = b->route_ids + (size_t)l * kBdMaxSeqs * 8;
        m.weights = b->route_w + (size_t)l * kBdMaxSeqs * 8;
        m.mutant = knobs().moe_mutant;
        m.errc = &b->io->moe_late;
        m.epoch_dev = &b->io->plan_epoch;
        m.epoch_sub = l;
        m.plan_spins = m.mutant == 9 ? 0u : kMoePlanSpins;
        m.defer_combine = 1;  // the next layer's rows launch (or the final norm) adds the MoE rows
        OMEGA_HIP(F_SESSION, launch_moe_batch(m, st));
        a.moe_dp = m.dp;
        a.moe_row = m.pair_row;
        a.moe_w = m.weights;
        a.moe_mutant = m.mutant;
    }
    a.norm_w = b->final_norm;
    OMEGA_LAUNCH(k_bd_final, dim3(T), dim3(256), 0, st, a);
    LmArgs la;
    la.wt = b->lm->wt;
    la.n = b->lm->n;
    la.k = b->lm->k;
    la.hi = b->hid_hi;
    la.lo = b->hid_lo;
    la.T = T;
    la.logits = b->keep_logits ? b->logits : nullptr;
    la.argmax = &b->io->argmax[0][0];
    OMEGA_HIP(F_SESSION, launch_bd_lm(la, st));
    return OMEGA_GPU_OK;
}

bool fp8_is(const OmegaGpuFp8Tensor *t, uint32_t experts, uint32_t n, uint32_t k) {
    return t && t->experts == experts && t->n == n && t->k == k;
}

// After the step's copy back: the next tokens, or an error when a MoE planner's wait ran out (that
// layer's MoE rows, the step's later K/V rows and its logits are not the model's: the caller runs
// the step again)
int bd_finish(const BdIo *p, uint32_t seqs, uint32_t *next_tokens) {
    if (p->moe_late) {
        set_error(F_SESSION, "batch decode step: %u MoE plans timed out waiting for their rankings",
                  p->moe_late);
        return OMEGA_GPU_CHIP_FAIL;
    }
    for (uint32_t s = 0; s < seqs; ++s) next_tokens[s] = argmax_from_slots(p->argmax[s]);
    return OMEGA_GPU_OK;
}

}  // namespace

extern "C" {

int omega_gpu_batch_decode_create(const OmegaGpuBatchDecodeConfig *cfg, OmegaGpuBatchDecode **out) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (out) *out = nullptr;
    if (!cfg || !out || !cfg->router || !cfg->lm_head || !cfg->embed || !cfg->pool) {
        set_error(F_SESSION, "batch decode create: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    if (cfg->layers == 0 || cfg->layers > 64 || cfg->max_seqs == 0 || cfg->max_seqs > kBdMaxSeqs ||
        cfg->max_blocks_per_seq == 0 || cfg->max_pos == 0 || cfg->max_pos > cfg->max_blocks_per_seq * 16u) {
        set_error(F_SESSION,
                  "batch decode: layers %u (1..=64), max_seqs %u (1..=%u), max_blocks_per_seq %u, max_pos %u "
                  "(<= 16 x max_blocks_per_seq)",
                  cfg->layers, cfg->max_seqs, kBdMaxSeqs, cfg->max_blocks_per_seq, cfg->max_pos);
        return OMEGA_GPU_BAD_ARGS;
    }
    OmegaGpuRouter *r = static_cast<OmegaGpuRouter *>(cfg->router);
    OmegaGpuBf16Tensor *lm = static_cast<OmegaGpuBf16Tensor *>(cfg->lm_head);
    OmegaGpuBf16Tensor *em = static_cast<OmegaGpuBf16Tensor *>(cfg->embed);
    if (router_layers(r) < cfg->layers || router_rows(r) != 128 || lm->k != kBdH || em->k != kBdH ||
        lm->n != cfg->vocab || em->n != cfg->vocab || cfg->vocab % 16 != 0) {
        set_error(F_SESSION,
                  "batch decode: router (128 experts, >= %u layers), lm_head and embedding [%u][2048] "
                  "(vocab a multiple of 16) required",
                  cfg->layers, cfg->vocab);
        return OMEGA_GPU_BAD_ARGS;
    }
    const OmegaGpuKvLayout &lay = cfg->layout;
    if (lay.block_size != 16 || lay.num_layers < cfg->layers || lay.head_stride_bytes < 256 ||
        lay.token_stride_bytes < 4 * lay.head_stride_bytes ||
        lay.kv_plane_stride_bytes < 16 * lay.token_stride_bytes) {
        set_error(F_SESSION, "batch decode: the pool layout must hold 16-token pages of 4 kv heads x 128 bf16 "
                             "for every layer");
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *cx = ctx(F_SESSION);
    if (!cx) return OMEGA_GPU_CHIP_FAIL;
    int rc = bf16_ensure_tiled(F_SESSION, lm);
    if (rc) return rc;
    OmegaGpuBatchDecode *b = new OmegaGpuBatchDecode();
    b->cfg = *cfg;
    b->router = r;
    b->lm = lm;
    b->embed = em;
    b->g = geom_of(lay);
    b->layers.resize(cfg->layers);
    const uint32_t T = cfg->max_seqs;
    hipError_t e = hipSuccess;
    auto M = [&](void **p, size_t bytes) {
        if (e == hipSuccess) e = dev_malloc(p, bytes);
        if (e == hipSuccess) e = hipMemset(*p, 0, bytes);
    };
    M((void **)&b->x, (size_t)T * kBdH * 4);
    M((void **)&b->xq, (size_t)T * (kBdH / 128) * kTerms * 128);
    M((void **)&b->xs, (size_t)T * (kBdH / 128) * 16);
    M((void **)&b->qkv_part, (size_t)kDenseSlices * T * kBdQkv * 4);
    M((void **)&b->q, (size_t)T * 32 * 128 * 4);
    M((void **)&b->apart, (size_t)kItemMax * 32 * kPartStride * 4);
    M((void **)&b->oq, (size_t)T * 32 * kTerms * 128);
    M((void **)&b->os, (size_t)T * 32 * 16);
    M((void **)&b->o_part, (size_t)kDenseSlices * T * kBdH * 4);
    M((void **)&b->sink, 256);
    M((void **)&b->hidden, (size_t)T * kBdH * 4);
    M((void **)&b->hid_hi, (size_t)T * kBdH * 2);
    M((void **)&b->hid_lo, (size_t)T * kBdH * 2);
    M((void **)&b->logits, (size_t)T * cfg->vocab * 4);
    M((void **)&b->tables, (size_t)T * cfg->max_blocks_per_seq * 4);
    M(&b->moe, moe_work_bytes(T));
    M((void **)&b->route_ids, (size_t)cfg->layers * kBdMaxSeqs * 8 * 4);
    M((void **)&b->route_w, (size_t)cfg->layers * kBdMaxSeqs * 8 * 4);
    M((void **)&b->io, sizeof(BdIo));
    M((void **)&b->final_norm, kBdH * 4);
    M((void **)&b->rope_cos, (size_t)cfg->max_pos * 64 * 4);
    M((void **)&b->rope_sin, (size_t)cfg->max_pos * 64 * 4);
    for (auto &L : b->layers) {
        M((void **)&L.in_norm, kBdH * 4);
        M((void **)&L.q_norm, 128 * 4);
        M((void **)&L.k_norm, 128 * 4);
    }
    if (e == hipSuccess) e = host_malloc((void **)&b->pin, sizeof(BdIo), hipHostMallocDefault);
    if (e == hipSuccess) {
        std::vector<float> cs((size_t)cfg->max_pos * 64), sn((size_t)cfg->max_pos * 64);
        rope_table(cfg->rope_theta, cfg->max_pos, cs.data(), sn.data());
        e = hipMemcpy(b->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(b->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        set_error(F_SESSION, "batch decode create: %s", hipGetErrorString(e));
        omega_gpu_batch_decode_free(b);
        return OMEGA_GPU_CHIP_FAIL;
    }
    memset(b->pin, 0, sizeof(BdIo));
    *out = b;
    return OMEGA_GPU_OK;
}

void omega_gpu_batch_decode_free(OmegaGpuBatchDecode *b) {
    if (!b) return;
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    Ctx *c = ctx(F_SESSION);
    if (c) (void)hipStreamSynchronize(c->stream);
    for (auto &kv : b->exec) (void)hipGraphExecDestroy(kv.second);
    for (hipGraph_t gr : b->graphs) (void)hipGraphDestroy(gr);
    void *ps[] = {b->x, b->xq, b->xs, b->qkv_part, b->q, b->apart, b->oq, b->os, b->o_part, b->sink, b->hidden,
                  b->hid_hi, b->hid_lo, b->logits, b->tables, b->moe, b->route_ids, b->route_w, b->io,
                  b->final_norm, b->rope_cos, b->rope_sin};
    for (void *p : ps)
        if (p) (void)dev_free(p);
    for (auto &L : b->layers) {
        if (L.in_norm) (void)dev_free(L.in_norm);
        if (L.q_norm) (void)dev_free(L.q_norm);
        if (L.k_norm) (void)dev_free(L.k_norm);
    }
    if (b->pin) (void)host_free(b->pin);
    delete b;
}

int omega_gpu_batch_decode_set_layer(OmegaGpuBatchDecode *b, uint32_t layer, const void *qkv, const void *o,
                                     const void *gate_up, const void *down, const float *input_norm,
                                     const float *q_norm, const float *k_norm) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!b || !input_norm || !q_norm || !k_norm || layer >= b->cfg.layers) {
        set_error(F_SESSION, "batch decode set_layer: NULL pointer or layer out of range");
        return OMEGA_GPU_BAD_ARGS;
    }
    auto tq = static_cast<OmegaGpuFp8Tensor *>(const_cast<void *>(qkv));
    auto to = static_cast<OmegaGpuFp8Tensor *>(const_cast<void *>(o));
    auto tg = static_cast<OmegaGpuFp8Tensor *>(const_cast<void *>(gate_up));
    auto td = static_cast<OmegaGpuFp8Tensor *>(const_cast<void *>(down));
    if (!fp8_is(tq, 1, kBdQkv, kBdH) || !fp8_is(to, 1, kBdH, kBdAttn) || !fp8_is(tg, 128, 1536, kBdH) ||
        !fp8_is(td, 128, kBdH, 768)) {
        set_error(F_SESSION,
                  "batch decode layer %u: projections must be q|k|v 1x5120x2048, o 1x2048x4096, gate|up "
                  "128x1536x2048, down 128x2048x768",
                  layer);
        return OMEGA_GPU_BAD_ARGS;
    }
    int rc = fp8_ensure_tiled(F_SESSION, tq);
    if (!rc) rc = fp8_ensure_tiled(F_SESSION, to);
    if (!rc) rc = fp8_ensure_tiled(F_SESSION, tg);
    if (!rc) rc = fp8_ensure_tiled(F_SESSION, td);
    if (rc) return rc;
    BdLayer &L = b->layers[layer];
    L.qkv = tq;
    L.o = to;
    L.gu = tg;
    L.dn = td;
    OMEGA_HIP(F_SESSION, hipMemcpy(L.in_norm, input_norm, kBdH * 4, hipMemcpyHostToDevice));
    OMEGA_HIP(F_SESSION, hipMemcpy(L.q_norm, q_norm, 128 * 4, hipMemcpyHostToDevice));
    OMEGA_HIP(F_SESSION, hipMemcpy(L.k_norm, k_norm, 128 * 4, hipMemcpyHostToDevice));
    return OMEGA_GPU_OK;
}

int omega_gpu_batch_decode_set_final_norm(OmegaGpuBatchDecode *b, const float *final_norm) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!b || !final_norm) {
        set_error(F_SESSION, "batch decode set_final_norm: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    OMEGA_HIP(F_SESSION, hipMemcpy(b->final_norm, final_norm, kBdH * 4, hipMemcpyHostToDevice));
    b->final_set = true;
    return OMEGA_GPU_OK;
}

int omega_gpu_batch_decode_set_tables(OmegaGpuBatchDecode *b, uint32_t seqs, const int32_t *tables) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!b || !tables || seqs == 0 || seqs > b->cfg.max_seqs) {
        set_error(F_SESSION, "batch decode set_tables: NULL pointer or %u sequences", seqs);
        return OMEGA_GPU_BAD_ARGS;
    }
    const size_t n = (size_t)seqs * b->cfg.max_blocks_per_seq;
    for (size_t i = 0; i < n; ++i) {
        if (tables[i] < -1 || tables[i] >= (int32_t)b->cfg.layout.num_blocks) {
            set_error(F_SESSION, "batch decode set_tables: entry %zu is %d (pool has %u blocks)", i, tables[i],
                      b->cfg.layout.num_blocks);
            return OMEGA_GPU_BAD_ARGS;
        }
    }
    Ctx *c = ctx(F_SESSION);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    OMEGA_HIP(F_SESSION, hipStreamSynchronize(c->stream));
    OMEGA_HIP(F_SESSION, hipMemcpy(b->tables, tables, n * 4, hipMemcpyHostToDevice));
    b->table_pages.assign(b->cfg.max_seqs, 0);
    for (uint32_t q = 0; q < seqs; ++q) {
        uint32_t k = 0;
        while (k < b->cfg.max_blocks_per_seq && tables[(size_t)q * b->cfg.max_blocks_per_seq + k] >= 0) ++k;
        b->table_pages[q] = k;
    }
    b->tables_set = true;
    return OMEGA_GPU_OK;
}

void omega_gpu_batch_decode_set_keep_logits(OmegaGpuBatchDecode *b, int on) {
    if (!b) return;
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    b->keep_logits = on != 0;
}

void omega_gpu_batch_decode_set_eager(OmegaGpuBatchDecode *b, int on) {
    if (!b) return;
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    b->eager = on != 0;
}

int omega_gpu_batch_decode_step(OmegaGpuBatchDecode *b, uint32_t seqs, const uint32_t *tokens,
                                const uint32_t *positions, uint32_t *next_tokens) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!b || !tokens || !positions || !next_tokens || seqs == 0 || seqs > b->cfg.max_seqs) {
        set_error(F_SESSION, "batch decode step: NULL pointer or %u sequences", seqs);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (!b->final_set || !b->tables_set) {
        set_error(F_SESSION, "batch decode step: final norm or page tables not set");
        return OMEGA_GPU_BAD_ARGS;
    }
    for (uint32_t l = 0; l < b->cfg.layers; ++l)
        if (!b->layers[l].qkv) {
            set_error(F_SESSION, "batch decode step: layer %u has no projections", l);
            return OMEGA_GPU_BAD_ARGS;
        }
    BdIo *p = b->pin;
    memset(p, 0, sizeof(BdIo));
    uint32_t total = 0;
    uint32_t first[kBdMaxSeqs + 1];  // the sequences' pages laid end to end
    for (uint32_t s = 0; s < seqs; ++s) {
        if (positions[s] >= b->cfg.max_pos) {
            set_error(F_SESSION, "batch decode step: sequence %u position %u >= max_pos %u", s, positions[s],
                      b->cfg.max_pos);
            return OMEGA_GPU_BAD_ARGS;
        }
        // every page up to the token's own must be named by the table (the kernels read them all)
        if (positions[s] / 16 >= b->table_pages[s]) {
            set_error(F_SESSION, "batch decode step: sequence %u position %u needs page %u, its table names %u",
                      s, positions[s], positions[s] / 16, b->table_pages[s]);
            return OMEGA_GPU_BAD_ARGS;
        }
        p->tok[s] = tokens[s];
        p->pos[s] = positions[s];
        first[s] = total;
        total += (positions[s] + 1 + 15) / 16;
    }
    first[seqs] = total;
    plan_items(first, seqs, p->plan);
    Ctx *c = ctx(F_SESSION);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    if (plan_epoch_take(F_SESSION, c->stream, &p->plan_epoch)) return OMEGA_GPU_CHIP_FAIL;
    if (b->eager) {
        OMEGA_HIP(F_SESSION, hipMemcpyAsync(b->io, p, sizeof(BdIo), hipMemcpyHostToDevice, c->stream));
        int rc = bd_enqueue(b, seqs, c->stream);
        if (rc) return rc;
        OMEGA_HIP(F_SESSION, hipMemcpyAsync(&p->moe_late, &b->io->moe_late, bd_back_bytes(seqs),
                                            hipMemcpyDeviceToHost, c->stream));
        OMEGA_HIP(F_SESSION, hipStreamSynchronize(c->stream));
        return bd_finish(p, seqs, next_tokens);
    }
    // the recorded launches carry the MoE test mutant they were recorded with
    const uint32_t key = seqs | (b->keep_logits ? 256u : 0u) | ((uint32_t)knobs().moe_mutant << 9);
    auto it = b->exec.find(key);
    if (it == b->exec.end()) {
        // built node by node (no stream capture)
        hipGraph_t graph = nullptr;
        hipGraphExec_t ex = nullptr;
        const int rc = build_graph(F_SESSION, "batch decode graph", &graph, &ex,
                                   [&]() { return bd_enqueue(b, seqs, c->stream); });
        if (rc) return rc;
        b->graphs.push_back(graph);
        it = b->exec.emplace(key, ex).first;
    }
    OMEGA_HIP(F_SESSION, hipMemcpyAsync(b->io, p, sizeof(BdIo), hipMemcpyHostToDevice, c->stream));
    OMEGA_HIP(F_SESSION, hipGraphLaunch(it->second, c->stream));
    OMEGA_HIP(F_SESSION, hipMemcpyAsync(&p->moe_late, &b->io->moe_late, bd_back_bytes(seqs),
                                        hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_SESSION, hipStreamSynchronize(c->stream));
    return bd_finish(p, seqs, next_tokens);
}

int omega_gpu_batch_decode_read(OmegaGpuBatchDecode *b, uint32_t seqs, float *x, float *hidden, float *logits,
                                uint32_t *route_ids) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!b || seqs == 0 || seqs > b->cfg.max_seqs) {
        set_error(F_SESSION, "batch decode read: NULL handle or %u sequences", seqs);
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *c = ctx(F_SESSION);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    OMEGA_HIP(F_SESSION, hipStreamSynchronize(c->stream));
    if (x) OMEGA_HIP(F_SESSION, hipMemcpy(x, b->x, (size_t)seqs * kBdH * 4, hipMemcpyDeviceToHost));
    if (hidden) OMEGA_HIP(F_SESSION, hipMemcpy(hidden, b->hidden, (size_t)seqs * kBdH * 4, hipMemcpyDeviceToHost));
    if (logits) {
        if (!b->keep_logits) {
            set_error(F_SESSION, "batch decode read: logits are kept only with set_keep_logits(1)");
            return OMEGA_GPU_BAD_ARGS;
        }
        OMEGA_HIP(F_SESSION, hipMemcpy(logits, b->logits, (size_t)seqs * b->cfg.vocab * 4, hipMemcpyDeviceToHost));
    }
    if (route_ids)
        for (uint32_t l = 0; l < b->cfg.layers; ++l)
            OMEGA_HIP(F_SESSION, hipMemcpy(route_ids + (size_t)l * seqs * 8, b->route_ids + (size_t)l * kBdMaxSeqs * 8,
                                           (size_t)seqs * 8 * 4, hipMemcpyDeviceToHost));
    return OMEGA_GPU_OK;
}

}  // extern "C"
