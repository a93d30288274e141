// Kernel argument blocks and host-side launchers shared by the ABI entry points and the decode
// graph. Every launcher enqueues on the given stream and returns the launch status; the
// launchers validate nothing (the entry points check shapes before they call them).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace omega {

// The KV of the paged pool (aien-kv-cache): element (block, layer, plane, token, head, dim) at
// block*BS + layer*LS + plane*PS + token*TS + head*HS + dim*2, bf16. The fused decode cache uses
// the same pages with the identity block table, but its V plane is stored transposed per page:
// element (token, head, dim) of V at plane + head*4096 + dim*32 + (token % 16)*2.
struct KvGeom {
    uint64_t block_stride, layer_stride, plane_stride, token_stride, head_stride;
    uint32_t block_size;
};

// ---------------------------------------------------------------- FP8 GEMV (row-major)
enum Fp8Epi : int {
    EPI_STORE = 0,  // y[g][r] = v
    EPI_RESID = 1,  // y[r] += v          (o_proj into the residual row)
};
enum XSrc : int {
    XS_F32 = 0,         // x (f32, group g at x + g * x_stride)
    XS_NORM = 1,        // RMSNorm(x) * norm_w   (k = 2048)
    XS_EMBED_NORM = 2,  // x = bf16 embedding row *embed_tok % embed_rows, then RMSNorm
};

struct Fp8RowsArgs {
    const uint8_t *w = nullptr;     // tensor base (expert 0), row-major [experts][n][k]
    const float *s = nullptr;       // f32 scales [experts][n/128][k/128]
    const uint64_t *tab = nullptr;  // device group table {w_va, s_va} x groups, or null
    const float *x = nullptr;
    uint32_t x_stride = 0;
    float x_scale = 1.0f;           // applied to the row sums (exact power of two)
    const float *norm_w = nullptr;
    float eps = 1e-6f;
    const uint16_t *embed = nullptr;     // XS_EMBED_NORM
    const uint32_t *embed_tok = nullptr;
    uint32_t embed_rows = 0;
    float *x_out = nullptr;         // XS_EMBED_NORM: workgroup 0 stores the widened row here
    uint32_t n = 0, k = 0, groups = 1;
    float *y = nullptr;
    int mutant = 0;                 // omega_gpu_fp8_test_set_mutant
    uint32_t ids[64] = {0};         // expert id per group when tab == null
};
hipError_t launch_fp8_rows(const Fp8RowsArgs &a, int epi, int xsrc, hipStream_t st);
uint32_t fp8_rows_per_wave(uint32_t k);
uint32_t fp8_rows_blocks(const Fp8RowsArgs &a);

hipError_t launch_fp8_tile(const uint8_t *w, uint8_t *wt, uint32_t experts, uint32_t n, uint32_t k,
                           hipStream_t st);
hipError_t launch_fp8_synth(uint8_t *w, float *s, uint32_t experts, uint32_t n, uint32_t k,
                            uint64_t seed, uint64_t tensor, float sigma, hipStream_t st);
// sets *flag when any byte is an e4m3 NaN (0x7f / 0xff)
hipError_t launch_fp8_nan_scan(const uint8_t *w, size_t bytes, uint32_t *flag, hipStream_t st);

// ---------------------------------------------------------------- bf16 GEMV (+ argmax)
struct Bf16RowsArgs {
    const uint16_t *w = nullptr;  // row-major [n][k]
    uint32_t n = 0, k = 0;
    const float *x = nullptr;
    const float *norm_w = nullptr;  // RMSNorm(x) first (k = 2048)
    float eps = 1e-6f;
    float *hidden_out = nullptr;    // with norm_w: workgroup 0 stores the normed row here
    float *y = nullptr;
    unsigned long long *argmax = nullptr;  // [kArgmaxSlots] packed (value, ~index) maxima
    int mutant = 0;
};
constexpr uint32_t kArgmaxSlots = 64;
hipError_t launch_bf16_rows(const Bf16RowsArgs &a, hipStream_t st);
hipError_t launch_bf16_synth(uint16_t *w, uint32_t n, uint32_t k, uint64_t seed, uint64_t tensor,
                             float sigma, hipStream_t st);
// `count` bf16 values of the same generator into any device buffer
hipError_t launch_bf16_synth_count(uint16_t *w, size_t count, uint64_t seed, uint64_t tensor, float sigma,
                                   hipStream_t st);
// sets *flag when any element is NaN or infinite
hipError_t launch_bf16_scan(const uint16_t *w, size_t count, uint32_t *flag, hipStream_t st);
// host side of the argmax: the greedy token from the slots (lowest index of the maximum)
uint32_t argmax_from_slots(const unsigned long long *slots);

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
    float *logits = nullptr;          // [rows]
    float *xout = nullptr;            // [hidden] x' * out_scale
    uint32_t *ids = nullptr;          // [slots]
    float *weights = nullptr;         // [slots]
    uint64_t *tab_gu = nullptr;       // [slots][2]
    uint64_t *tab_dn = nullptr;
    uint32_t *route_log = nullptr;    // optional copies of ids / weights (decode graph log)
    float *route_log_w = nullptr;
    int mutant = 0;
};
// logits (and x'); then the ranking of the logits (ids, weights, group tables)
hipError_t launch_router_logits(const RouterArgs &a, hipStream_t st);
hipError_t launch_router_topk(const RouterArgs &a, hipStream_t st);
// one token's MoE block through the decode step's kernels (router logits, gate|up with the
// ranking in its prologue, down with the combine): three launches
hipError_t launch_moe_one_token(const RouterArgs &ra, const uint8_t *gu_w, const float *gu_s,
                                const uint8_t *dn_w, const float *dn_s, float *act, const float *resid,
                                float *out, hipStream_t st);

// ---------------------------------------------------------------- attention
constexpr uint32_t kAttnTile = 64;       // tokens per tile of the paged kernel (one wavefront)
constexpr uint32_t kDattnPage = 16;      // tokens per split unit of the fused kernel (one page)
constexpr uint32_t kDattnSplits = 64;    // split workgroups per kv head of the fused kernel
constexpr uint32_t kPartStride = 132;    // floats per (head, split) partial: m, l, -, -, o[128]

// How `tiles` tiles of 64 tokens spread over at most `splits` split items: `tps` tiles each
// (forced_tps when non-zero and it fits), `active` items hold work; with no tiles one item still
// runs (the fused kernel folds the current token into split 0).
__host__ __device__ inline void attn_split_plan(uint32_t tiles, uint32_t splits, uint32_t forced_tps,
                                                uint32_t &active, uint32_t &tps) {
    if (tiles == 0) {
        active = 1;
        tps = 0;
        return;
    }
    tps = forced_tps ? forced_tps : (tiles + splits - 1) / splits;
    if ((tiles + tps - 1) / tps > splits) tps = (tiles + splits - 1) / splits;
    active = (tiles + tps - 1) / tps;
}

// Fused decode attention over the cache: per (split, kv head) one wavefront prepares the 8 q
// heads (RMSNorm, RoPE) from the raw q|k|v row, runs the matrix-core flash-decoding of its tiles
// of the tokens before `pos`, and split 0 also appends this token's K/V and folds it in.
constexpr uint32_t kDattnMergeSpins = 1u << 22;  // bounded wait of the split merge (seconds)
struct DattnArgs {
    const float *qkv = nullptr;      // raw q|k|v [5120]
    uint8_t *pool = nullptr;
    KvGeom g{};
    uint32_t layer = 0, max_pos = 0;
    const float *q_norm = nullptr, *k_norm = nullptr;      // [128] of the layer
    const float *rope_cos = nullptr, *rope_sin = nullptr;  // [max_pos][64]
    float eps = 1e-6f;
    const uint32_t *pos_dev = nullptr;
    uint32_t pos_host = 0;
    uint32_t tiles_per_split = 0;    // pages per split; 0: spread over every split
    float *part = nullptr;           // [32][kDattnSplits][kPartStride]
    // The split merge in the same launch: split s of kv head h, once its partial is stored, sets
    // flags[h * kDattnSplits + s] to this launch's epoch; splits 0..7 of a kv head then wait for
    // every split of the head and each merges q head 8 h + s into out. The epoch is unique per
    // launch among the launches that share `flags` (epoch_dev * 64 + layer, or epoch_host when
    // epoch_dev is null); *errc counts waits that ran out of spins.
    uint32_t *flags = nullptr;       // [4 * kDattnSplits]
    uint32_t *errc = nullptr;
    const uint32_t *epoch_dev = nullptr;
    uint32_t epoch_host = 0;
    float *out = nullptr;            // [32][128]
    float out_scale = 1.0f;
    int mutant = 0;  // 1: no RoPE; 2: V written one position late; 3: K/V not written; 4: maxima ignored
    uint32_t splits = kDattnSplits;  // split workgroups per kv head (the launch's grid y, <= kDattnSplits)
    uint32_t merge_spins = kDattnMergeSpins;  // the merge's bounded wait; 0: gives up at once (counted)
};
// The decode graph cuts a kv head's pages into at most this many splits in both of its forms (the
// persistent launch holds two splits per attention workgroup), so the two forms give the same bits
// at every position.
constexpr uint32_t kGraphSplits = 64;
hipError_t launch_dattn(const DattnArgs &a, hipStream_t st);

// Paged flash-decoding over an external pool: grid (splits, kv heads, seqs), one wavefront
// per item, partials as above.
struct AttnArgs {
    const float *q = nullptr;               // [seqs][qh][128] post-norm, post-rope
    const uint8_t *pool = nullptr;
    KvGeom g{};
    uint32_t layer = 0;
    const int32_t *block_tables = nullptr;  // [seqs][max_blocks]
    uint32_t max_blocks = 0;
    const int32_t *context_lens = nullptr;  // [seqs]
    uint32_t seqs = 1, qh = 32, kvh = 4;
    uint32_t splits = 1;
    float *part = nullptr;                  // [seqs][qh][splits][kPartStride]
    int mutant = 0;                         // 2: V one position late; 4: merge ignores the maxima
    // the folded form (the split merge in the same launch): out, the (sequence, split) flags,
    // this launch's epoch, the merge's bounded wait (0: gives up at once) and its give-up count
    float *out = nullptr;                   // [seqs][qh][128]
    float out_scale = 1.0f;
    uint32_t *flags = nullptr;
    uint32_t *errc = nullptr;
    uint32_t epoch = 0;
    uint32_t merge_spins = kDattnMergeSpins;
    uint32_t ctx_hint = 0;  // the call's longest context: the split plan the page ids are read for early
};
hipError_t launch_attention(const AttnArgs &a, hipStream_t st);
// GQA group 8 over 16-token pages runs on the matrix cores (k_paged), other shapes on the VALU
bool paged_mfma(uint32_t qh, uint32_t kvh, uint32_t block_size);
uint32_t paged_splits(uint32_t max_ctx, uint32_t seqs, uint32_t kvh, bool mfma, uint32_t &unit);

// Combines the split partials of every (seq, q head): out = sum w_s o_s / sum w_s l_s with
// w_s = exp(m_s - max m), times out_scale.
struct CombineArgs {
    const float *part = nullptr;
    uint32_t splits = 1;                    // partial slots per head
    const uint32_t *pos_dev = nullptr;      // fused: tiles before pos, plus the token itself
    uint32_t pos_host = 0;
    uint32_t tiles_per_split = 0;           // as the fused kernel's
    uint32_t tile_tokens = kAttnTile;       // tokens per split unit (kDattnPage for the fused kernel)
    const int32_t *context_lens = nullptr;  // paged: tiles of the context
    uint32_t seqs = 1, qh = 32;
    float out_scale = 1.0f;
    float *out = nullptr;                   // [seqs][qh][128]
    int mutant = 0;                         // 4: ignore the maxima
};
hipError_t launch_attn_combine(const CombineArgs &a, hipStream_t st);

// ---------------------------------------------------------------- batched MoE block
// T tokens (<= kMoeMaxTokens) through RMSNorm, router logits, top-8 and grouping, the grouped
// gate|up (SwiGLU) and down FP8 GEMMs on the matrix cores, and the slot-order combine.
constexpr uint32_t kMoeMaxTokens = 64;
// below this token count the expert projections run as grouped GEMVs on f32 activations (each
// segment's weights held in registers across its rows); from it on, on the FP8 matrix cores
constexpr uint32_t kMoeGemvMax = 16;
constexpr uint32_t kMoePlanSpins = 1u << 22;  // bounded wait of the planner (seconds)
struct MoeArgs {
    const float *h = nullptr;          // [T][2048] residual rows
    const float *norm_w = nullptr;     // post-attention RMSNorm weights [2048]
    const uint16_t *gate = nullptr;    // router [128][2048] bf16
    float eps = 1e-6f;
    int norm_topk = 1;
    uint32_t tokens = 0;
    const uint8_t *gu_wt = nullptr;    // [128][1536][2048] e4m3, tiled twin
    const float *gu_s = nullptr;       // [128][12][16]
    const uint8_t *dn_wt = nullptr;    // [128][2048][768] e4m3, tiled twin
    const float *dn_s = nullptr;       // [128][16][6]
    const uint8_t *gu_w = nullptr;     // the row-major bytes (the GEMV path, tokens < kMoeGemvMax)
    const uint8_t *dn_w = nullptr;
    const float *resid = nullptr;      // optional: out = resid + moe
    const float *opart = nullptr;      // optional: h += sum of oslices k-slices [oslices][T][2048]
    uint32_t oslices = 0;              //   (the o projection's partials), stored to hout
    float *hout = nullptr;
    uint32_t *ids = nullptr;           // [T][8]
    float *weights = nullptr;          // [T][8]
    float *out = nullptr;              // [T][2048]
    // workspace (moe_work_carve)
    float *xn = nullptr;               // [T][2048] x'
    uint8_t *xq = nullptr;             // [T][16][4][128] e4m3 terms of x'
    float *xs = nullptr;               // [T][16][4] their scales
    float *logits = nullptr;           // [T][128]
    uint32_t *plan = nullptr;          // [0]: segments, [1]: 1 when the planner's wait ran out
    uint32_t *errc = nullptr;          // optional: counts the planner's waits that ran out
    // the planner's launch epoch (its flags carry it): *epoch_dev * 64 + epoch_sub when epoch_dev
    // is set (a word the host writes before each replay of a recorded graph), else epoch_host;
    // every launch on the device takes a value no earlier launch used (plan_epoch_take)
    const uint32_t *epoch_dev = nullptr;
    uint32_t epoch_sub = 0;
    uint32_t epoch_host = 0;
    uint32_t plan_spins = kMoePlanSpins;  // the planner's bounded wait; 0: gives up at once
    int defer_combine = 0;             // 1: no combine launch; the caller adds the dp rows
    uint32_t *seg_expert = nullptr, *seg_start = nullptr, *seg_count = nullptr;  // [128]
    uint32_t *pair_row = nullptr;      // [T * 8]: grouped row of pair t * 8 + s
    uint32_t *row_token = nullptr;     // [T * 8]: token of grouped row
    float *gp = nullptr;               // [T * 8][768] SwiGLU rows (the GEMV path)
    uint8_t *aq = nullptr;             // [T * 8][6][4][128] split terms of the SwiGLU rows
    float *as = nullptr;               // [T * 8][6][4]
    float *dp = nullptr;               // [T * 8][2048] down rows
    int mutant = 0;  // 1: rank mask id^1; 2: weights not normalised; 5: gate/up swapped;
                     // 6: slot 7 dropped; 7: one activation term; 9: the planner's wait gives up
                     // at once (plan_spins 0)
};
hipError_t launch_moe_batch(const MoeArgs &a, hipStream_t st);
// A fresh planner epoch base for the next launch(es) on the device's stream st: launches use
// base * 64 + sub with sub < 64, or base * 64. Before the bases wrap the flags are cleared on st
// and the bases start again from 1. Call outside graph recording (it may enqueue a memset).
int plan_epoch_take(int family, hipStream_t st, uint32_t *base);  // family: an omega::Family
size_t moe_work_carve(MoeArgs &a, void *base, uint32_t tokens);
size_t moe_work_bytes(uint32_t tokens);

// ---------------------------------------------------------------- batched decode attention
// Ragged paged attention (GQA 32 q / 4 kv heads over 16-token pages, the matrix-core page loop):
// item i is split i - item_off[s] of sequence s, pages [split * pps[s], +pps[s]) of its pos[s] + 1
// tokens; partials at part[(i * 32 + q head) * kPartStride].
// The attention work of a batched decode step over ragged sequences: the sequences' pages laid
// end to end are cut into kItemRuns equal runs, one per workgroup of four wavefronts (one per
// kv head; 512 x 4 = 2048 = 256 CUs x 8, the paged kernel's occupancy of 2 per SIMD: every
// wavefront is resident at once and they all finish together), and each run into items at
// sequence boundaries.
constexpr uint32_t kItemRuns = 512;
constexpr uint32_t kItemMaxSeqs = 32;
constexpr uint32_t kItemMax = kItemRuns + kItemMaxSeqs;  // items of a step at most
struct ItemPlan {
    uint32_t item_off[kItemMaxSeqs + 1];  // items of sequence s: [item_off[s], item_off[s + 1])
    uint32_t pad[3];
    uint32_t run_off[kItemRuns + 4];      // items of run (workgroup) r: [run_off[r], run_off[r + 1])
    uint32_t items[kItemMax][2];          // {seq << 24 | first page, end page}
};
// first[s] .. first[s + 1]: sequence s's pages laid end to end (every sequence has >= 1 page)
void plan_items(const uint32_t *first, uint32_t seqs, ItemPlan &p);

struct PagedItemsArgs {
    const float *q = nullptr;            // [seqs][32][128] post-norm, post-RoPE
    const uint8_t *pool = nullptr;
    KvGeom g{};
    uint32_t layer = 0;
    const int32_t *tables = nullptr;     // [seqs][max_blocks]
    uint32_t max_blocks = 0;
    const uint32_t *pos = nullptr;       // [seqs]
    const uint32_t *run_off = nullptr;  // [runs + 1]: items of workgroup r
    const uint32_t *items = nullptr;     // [items][2]: {seq << 24 | first page, end page}
    float *part = nullptr;               // [items][32][kPartStride]
};
hipError_t launch_paged_items(const PagedItemsArgs &a, uint32_t runs, hipStream_t st);
// the items' partials of every (seq, q head) combined (at most kCombineMaxItems items per
// sequence) and split into the o projection's input terms: oq [seqs][32][4][128] e4m3,
// os [seqs][32][4]
constexpr uint32_t kCombineMaxItems = 768;
static_assert(kItemRuns <= kCombineMaxItems, "a sequence may get an item from every wavefront");
struct CombineItemsArgs {
    const float *part = nullptr;
    const uint32_t *item_off = nullptr;  // [seqs + 1]: items of sequence s
    uint8_t *oq = nullptr;
    float *os = nullptr;
    float *out = nullptr;                // when set: the f32 rows [seqs][32][128] instead of the split
    float out_scale = 1.0f;              // the f32 rows' factor
};
hipError_t launch_attn_combine_items(const CombineItemsArgs &a, uint32_t seqs, hipStream_t st);

// RoPE table of one position range (host twin of the oracle's rope_cos_sin)
void rope_table(double theta, uint32_t positions, float *cos_out, float *sin_out);

// ---------------------------------------------------------------- persistent decode token
// The decode graph's layers as one persistent launch (ptoken.hip). One descriptor per layer, in
// device memory.
struct PLayer {
    const uint8_t *qkv_w;  // [5120][2048] e4m3, scales [40][16]
    const float *qkv_s;
    const uint8_t *o_w;    // [2048][4096], scales [16][32]
    const float *o_s;
    const uint8_t *gu_w;   // [128][1536][2048], scales [128][12][16]
    const float *gu_s;
    const uint8_t *dn_w;   // [128][2048][768], scales [128][16][6]
    const float *dn_s;
    const float *in_norm;  // [2048]
    const uint16_t *rgate; // router [128][2048] bf16
    const float *rnorm;    // [2048]
    const uint64_t *dir_gu, *dir_dn;  // [128][2]: expert weight / scale addresses
    const float *q_norm, *k_norm;     // [128]
    const uint32_t *forced;           // parity tests: 8 expert ids instead of the ranking, or null
    uint32_t *log_ids;                // [8] routed ids of the last token
    float *log_w;                     // [8]
};
constexpr uint32_t kTokGroups = 256;   // one workgroup per CU, all resident
constexpr uint32_t kTokThreads = 512;  // eight wavefronts
constexpr uint32_t kTokStampsPerLayer = 5;
struct PTokenArgs {
    const PLayer *layers = nullptr;
    uint32_t nlayers = 0;
    const uint32_t *io = nullptr;  // pos, token id, epoch (written by the host before the launch)
    uint32_t *errc = nullptr;      // waits that ran out
    uint32_t *abort = nullptr;     // set by the first wait that runs out: every later wait ends
    const uint16_t *embed = nullptr;  // layer 0's row from the embedding by token id, or null: from x
    uint32_t embed_rows = 0;
    float *x = nullptr;            // residual row: layer 0's input without embed; the last layer's output
    uint8_t *pool = nullptr;       // the fused decode cache
    KvGeom g{};
    uint32_t max_pos = 0;
    const float *rope_cos = nullptr, *rope_sin = nullptr;
    float eps = 1e-6f;
    int norm_topk = 1;
    // words (f32 value | epoch), one buffer per (layer, stage)
    uint64_t *w_x = nullptr;    // [layers + 1][2048] layer inputs (index 0 unused)
    uint64_t *w_qkv = nullptr;  // [layers][5120]
    uint64_t *w_att = nullptr;  // [layers][4096]
    uint64_t *w_xn = nullptr;   // [layers][2048] residual after the attention
    uint64_t *w_log = nullptr;  // [layers][128]
    uint64_t *w_xp = nullptr;   // [layers][2048] the post-attention normed row x'
    uint64_t *w_act = nullptr;  // [layers][8][768]
    float *part = nullptr;      // attention partials [32][kDattnSplits][kPartStride]
    uint32_t *aflags = nullptr; // [layers][4][kDattnSplits] split flags (epochs)
    // the router's device state after the token (the last layer's)
    float *r_xout = nullptr, *r_logits = nullptr, *r_weights = nullptr;
    uint32_t *r_ids = nullptr;
    uint64_t *r_tab_gu = nullptr, *r_tab_dn = nullptr;
    int graph_mutant = 0;       // 1: gate and up swapped; 2: slot 7 dropped from the combine
    uint64_t wait_ticks = 0;    // a wait runs out after this many 100 MHz ticks (0 runs out at once)
    int dattn_mutant = 0;
    int router_mutant = 0;
    uint32_t tiles_per_split = 0;
    float attn_out_scale = 1.0f;
    unsigned long long *stamps = nullptr;  // [1 + layers * kTokStampsPerLayer] or null
};
constexpr uint32_t kTokLds = 96 * 1024;  // dynamic LDS: one workgroup per CU
hipError_t launch_token(const PTokenArgs &a, hipStream_t st);
// whether this device can hold every workgroup of the persistent token kernel at once
bool token_fits(int device);

}  // namespace omega
