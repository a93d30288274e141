// Kernel argument blocks and host-side launchers shared by the ABI entry points and the decode
// graph. Every launcher enqueues on the given stream and returns the launch status; the
// launchers validate nothing (the entry points check shapes before they call them).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace omega {

// The KV of the fused cache and of the paged pool share one page layout (aien-kv-cache):
// element (block, layer, plane, token, head, dim) at block*BS + layer*LS + plane*PS + token*TS +
// head*HS + dim*2, bf16. The fused cache is a pool with the identity block table.
struct KvGeom {
    uint64_t block_stride, layer_stride, plane_stride, token_stride, head_stride;
    uint32_t block_size;
};

// Everything one head of the fused q|k|v row needs to be prepared (device.hpp prep_head).
struct HeadPrep {
    float *q_out = nullptr;          // [qh][128] post-norm, post-rope q
    uint8_t *pool = nullptr;         // page pool (identity block table)
    KvGeom g{};
    uint32_t layer = 0;
    const float *q_norm = nullptr, *k_norm = nullptr;      // [128]
    const float *rope_cos = nullptr, *rope_sin = nullptr;  // [max_pos][64]
    float eps = 1e-6f;
    uint32_t qh = 32, kvh = 4;
    int mutant = 0;                  // 1: no RoPE; 3: K/V not written
};

// ---------------------------------------------------------------- FP8 GEMV (row-per-lane)
enum Fp8Epi : int {
    EPI_STORE = 0,    // y[g][r] = v
    EPI_RESID = 1,    // y[r] += v          (o_proj into the residual row)
    EPI_SWIGLU = 2,   // y[g][j] = silu(v[j]) * v[n/2 + j]   (gate|up pairs -> activation)
    EPI_COMBINE = 3,  // y[r] += sum_g w[g] * v[g][r], slots in order (down -> MoE out + residual)
    EPI_QKV = 4,      // per 128-row head: q/k RMSNorm + RoPE -> q_out, K/V bf16 -> page pool
};

struct Fp8GemvArgs {
    const uint8_t *w = nullptr;   // tensor base (expert 0), tiled layout
    const float *s = nullptr;     // f32 scales base (expert 0)
    const uint64_t *tab = nullptr;  // device group table {w_va, s_va} x groups, or null
    const float *x = nullptr;     // activation; group g reads x + g * x_stride
    uint32_t x_stride = 0;
    float x_scale = 1.0f;         // folded into the block scales (exact power of two)
    const float *norm_w = nullptr;  // input RMSNorm weight (prologue), or null
    float eps = 1e-6f;
    uint32_t n = 0, k = 0, groups = 1, splits = 1;
    float *y = nullptr;
    float *partial = nullptr;     // [splits][groups][n] when splits > 1 or EPI_COMBINE
    uint32_t *counters = nullptr; // one per output tile, zero on entry, zero on exit
    const float *comb_w = nullptr;  // EPI_COMBINE slot weights (device)
    int mutant = 0;               // omega_gpu_fp8_test_set_mutant
    int graph_mutant = 0;         // omega_gpu_decode_graph_test_set_mutant (swiglu / combine)
    HeadPrep prep{};              // EPI_QKV
    const uint32_t *pos_dev = nullptr;  // EPI_QKV position (device), else pos_host
    uint32_t pos_host = 0;
    uint32_t ids[64] = {0};       // expert id per group when tab == null
};

// steps = 16-byte column steps per work item (8 or 16); the grid is computed from the args.
hipError_t launch_fp8_gemv(const Fp8GemvArgs &a, int steps, hipStream_t st);
hipError_t launch_fp8_gemv_epi(const Fp8GemvArgs &a, int steps, int epi, hipStream_t st);
// work items (= workgroups) a launch of these args uses
uint32_t fp8_gemv_items(const Fp8GemvArgs &a, int steps);
// choose the steps and splits for a shape (fills a.splits); returns steps
int fp8_gemv_plan(Fp8GemvArgs &a, int epi);

// upload helpers
hipError_t launch_fp8_relayout(const uint8_t *src, uint8_t *dst, uint32_t experts, uint32_t n,
                               uint32_t k, uint32_t *nan_flag, hipStream_t st);
hipError_t launch_fp8_synth(uint8_t *w, float *s, uint32_t experts, uint32_t n, uint32_t k,
                            uint64_t seed, uint64_t tensor, float sigma, hipStream_t st);

// ---------------------------------------------------------------- bf16 GEMV + argmax
struct Bf16GemvArgs {
    const uint16_t *w = nullptr;  // tiled layout, n_pad rows
    const float *x = nullptr;
    const float *norm_w = nullptr;  // optional RMSNorm of x first (final norm)
    float eps = 1e-6f;
    uint32_t n = 0, n_pad = 0, k = 0;
    float *y = nullptr;
    float *hidden_out = nullptr;    // when norm_w: the normed row is also written here
    // argmax (optional): per-tile partials and the result
    float *arg_val = nullptr;
    uint32_t *arg_idx = nullptr;
    uint32_t *token = nullptr;
    uint32_t *counter = nullptr;
    int mutant = 0;
};
hipError_t launch_bf16_gemv(const Bf16GemvArgs &a, hipStream_t st);
hipError_t launch_bf16_relayout(const uint16_t *src, uint16_t *dst, uint32_t n, uint32_t n_pad,
                                uint32_t k, uint32_t *bad_flag, hipStream_t st);
hipError_t launch_bf16_synth(uint16_t *w, uint32_t n, uint32_t n_pad, uint32_t k, uint64_t seed,
                             uint64_t tensor, float sigma, hipStream_t st);

// ---------------------------------------------------------------- router
struct RouterArgs {
    const float *x = nullptr;         // residual row [hidden]
    const uint16_t *gate = nullptr;   // [rows][hidden] bf16 (rows = experts + shared)
    const float *norm_w = nullptr;    // [hidden]
    const uint64_t *dir_gu = nullptr; // [rows][2]
    const uint64_t *dir_dn = nullptr;
    float eps = 1e-6f;
    int norm_topk = 1;
    float out_scale = 1.0f;
    uint32_t experts = 128, shared = 0, hidden = 2048, top_k = 8;
    float *logits = nullptr;          // [rows] scratch
    float *xout = nullptr;            // [hidden] x' * out_scale
    uint32_t *ids = nullptr;          // [slots]
    float *weights = nullptr;         // [slots]
    uint64_t *tab_gu = nullptr;       // [slots][2]
    uint64_t *tab_dn = nullptr;
    uint32_t *counter = nullptr;
    uint32_t *route_log = nullptr;    // optional: ids also written here (decode graph log)
    float *route_log_w = nullptr;     // optional: weights also written here
    int mutant = 0;
};
hipError_t launch_router(const RouterArgs &a, hipStream_t st);

// ---------------------------------------------------------------- attention

// Paged flash-decoding: grid (splits, kv heads, seqs), one wavefront per item; the tokens of a
// (seq, kv head) are cut into `splits` ranges of whole 64-token sub-chunks, each item keeps an
// online softmax over its range, and the last item of the (seq, kv head) combines the ranges in
// order. q is read wave-uniformly (scalar loads); K rows are read one per lane, V one dim pair
// per lane.
struct AttnArgs {
    const float *q = nullptr;               // [seqs][qh][128] post-norm, post-rope
    const uint8_t *pool = nullptr;          // page pool (device-readable)
    KvGeom g{};
    uint32_t layer = 0;
    const int32_t *block_tables = nullptr;  // [seqs][max_blocks]; null: identity (block = p/16)
    uint32_t max_blocks = 0;
    const int32_t *context_lens = nullptr;  // [seqs]; null: ctx = (*pos_dev or pos_host) + 1
    const uint32_t *pos_dev = nullptr;
    uint32_t pos_host = 0;
    uint32_t seqs = 1, qh = 32, kvh = 4;
    uint32_t splits = 1;                    // items per (seq, kv head)
    float out_scale = 1.0f;
    float *part = nullptr;                  // [seqs][qh][splits][132]: m, l, -, -, o[128]
    uint32_t *counters = nullptr;           // [seqs][kvh], zero on entry and exit
    float *out = nullptr;                   // [seqs][qh][128]
    int mutant = 0;                         // 2: V one position late; 4: combine ignores the max
};
hipError_t launch_attention(const AttnArgs &a, hipStream_t st);
// standalone preparation of a raw q|k|v row: one wavefront per head (qh + 2 kvh of them)
hipError_t launch_qkv_prep(const HeadPrep &p, const float *qkv, const uint32_t *pos_dev,
                           uint32_t pos_host, hipStream_t st);
// RoPE table of one position range (host twin of the oracle's rope_cos_sin)
void rope_table(double theta, uint32_t positions, float *cos_out, float *sin_out);

}  // namespace omega
