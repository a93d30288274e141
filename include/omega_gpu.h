/*
 * omega_gpu.h — the C ABI of the MI355X (gfx950) Qwen3-30B-A3B FP8 decode step.
 *
 * This library (libomega_gpu.so / libomega_gpu.a) is a drop-in for the external engine archive
 * the reference's Rust FFI crates link (aien-dev/aien-sovereign-core-mv, crates/aien-omega-*):
 * every declaration below has the symbol name, argument meaning, struct layout and return codes
 * the reference binds, and each cites the Rust `extern "C"` declaration it replaces
 * (file:line relative to the reference repository root). Plain pointers and sizes only.
 *
 * Conventions shared by every family (crates/aien-omega-gpu/src/ffi.rs:32-37):
 *   return 0 OK, -1 BAD_ARGS, -2 TOO_LARGE, -3 CODEGEN_FAIL, -4 CHIP_FAIL, -5 PARITY_FAIL /
 *   UNWRITTEN; *_rc_name(rc) returns a static string, *_last_error() a static string or NULL.
 *   Every call is synchronous: results are in host memory when it returns. Handles are used by
 *   one thread at a time; the library serialises its own global state with one lock.
 *   Upload and set calls copy the host buffers before they return.
 */
#ifndef OMEGA_GPU_H
#define OMEGA_GPU_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ return codes */
#define OMEGA_GPU_OK 0
#define OMEGA_GPU_BAD_ARGS (-1)
#define OMEGA_GPU_TOO_LARGE (-2)
#define OMEGA_GPU_CODEGEN_FAIL (-3)
#define OMEGA_GPU_CHIP_FAIL (-4)
#define OMEGA_GPU_PARITY_FAIL (-5)
#define OMEGA_GPU_UNWRITTEN (-5)

/* ================================================================== FP8 GEMV / GEMM
 * crates/aien-omega-fp8/src/lib.rs:16-29 (contract), :132-207 (declarations) */
#define OMEGA_GPU_FP8_BLOCK 128
#define OMEGA_GPU_FP8_MAX_GROUPS 64
#define OMEGA_FP8_MAX_K 32768
#define OMEGA_GPU_FP8GEMM_MAX_ROWS 1024
#define OMEGA_GPU_FP8GEMM_MAX_SEGMENTS 256

typedef struct OmegaGpuFp8Tensor OmegaGpuFp8Tensor;

/* fp8/src/lib.rs:94-116 (Rust mirror), layout asserted at :787-795 */
typedef struct OmegaGpuFp8Info {
    uint32_t experts, n, k, groups;
    uint32_t lane_bytes, rows_per_warp, warps_per_cta, depth;
    uint32_t grid_x, grid_y, steps;
    uint64_t weight_bytes;
    uint64_t scale_bytes;
    uint64_t elapsed_ns;
    uint64_t call_ns;
    uint32_t completion_marker;
    bool kernel_cache_hit;
    char target_chip[64];
    uint32_t sm_architecture;
} OmegaGpuFp8Info;

/* fp8/src/lib.rs:68-91, layout asserted at :797-810 */
typedef struct OmegaGpuFp8GemmInfo {
    uint32_t rows, segments, n, k, mt, warps_per_cta, lane_bytes, grid_x, grid_y, passes_max;
    uint64_t weight_bytes;
    uint64_t streamed_bytes;
    uint64_t elapsed_ns;
    uint64_t call_ns;
    uint32_t completion_marker;
    bool kernel_cache_hit;
} OmegaGpuFp8GemmInfo;

/* fp8/src/lib.rs:133-140: `experts` projections [expert][n][k] of e4m3 bytes plus bf16
 * weight_scale_inv [expert][n/128][k/128]. Refuses n%128, k%128, k outside 128..=32768, and any
 * e4m3 NaN code (0x7f / 0xff). */
int omega_gpu_fp8_tensor_upload(uint32_t experts, uint32_t n, uint32_t k, const uint8_t *w,
                                const uint16_t *scale_inv_bf16, OmegaGpuFp8Tensor **out);
/* fp8/src/lib.rs:141 */
void omega_gpu_fp8_tensor_free(OmegaGpuFp8Tensor *t);
/* fp8/src/lib.rs:142-148: y[n] = W[expert] x[k] */
int omega_gpu_fp8_gemv_f32(const OmegaGpuFp8Tensor *t, uint32_t expert, const float *x, float *y,
                           OmegaGpuFp8Info *info);
/* fp8/src/lib.rs:149-157: groups <= 64 experts; x is k values (x_rows 1) or groups*k; y is
 * groups*n, group-major */
int omega_gpu_fp8_gemv_grouped_f32(const OmegaGpuFp8Tensor *t, uint32_t groups,
                                   const uint32_t *expert_ids, const float *x, uint32_t x_rows,
                                   float *y, OmegaGpuFp8Info *info);
/* fp8/src/lib.rs:160-167: the group table ({w_va, s_va} x groups) and the activation row
 * (f32, pre-multiplied by 2^64) are device addresses the router wrote; y is unscaled */
int omega_gpu_fp8_gemv_grouped_dev(const OmegaGpuFp8Tensor *t, uint32_t groups, uint64_t tab_va,
                                   uint64_t x_va, float *y, OmegaGpuFp8Info *info);
/* fp8/src/lib.rs:168-173: device addresses of one expert's weights and scales */
int omega_gpu_fp8_tensor_entry(const OmegaGpuFp8Tensor *t, uint32_t expert, uint64_t *w_va,
                               uint64_t *s_va);
/* fp8/src/lib.rs:177-186: grouped GEMM over a row table sorted by expert; row i computes expert
 * expert_ids[i] on x[token_rows[i]]; y is m*n in row-table order. m <= 1024, <= 256 segments. */
int omega_gpu_fp8gemm_f32(const OmegaGpuFp8Tensor *t, uint32_t m, const uint32_t *expert_ids,
                          const uint32_t *token_rows, const float *x, uint32_t x_rows, float *y,
                          OmegaGpuFp8GemmInfo *info);
int omega_gpu_fp8gemm_prepare(uint32_t k);                 /* fp8/src/lib.rs:187 */
const char *omega_gpu_fp8gemm_rc_name(int rc);             /* fp8/src/lib.rs:188 */
const char *omega_gpu_fp8gemm_last_error(void);            /* fp8/src/lib.rs:189 */
void omega_gpu_fp8gemm_test_set_mutant(int mutant);        /* fp8/src/lib.rs:190 */
uint32_t omega_gpu_fp8_grouped_ctas_auto(uint32_t groups); /* fp8/src/lib.rs:194 */
int omega_gpu_fp8_prepare(uint32_t k);                     /* fp8/src/lib.rs:198 */
void omega_gpu_fp8_seal(int on);                           /* fp8/src/lib.rs:199 */
const char *omega_gpu_fp8_rc_name(int rc);                 /* fp8/src/lib.rs:200 */
const char *omega_gpu_fp8_last_error(void);                /* fp8/src/lib.rs:201 */
void omega_gpu_fp8_cache_clear(void);                      /* fp8/src/lib.rs:202 */
void omega_gpu_fp8_set_shape(uint32_t lane_bytes, uint32_t rows_per_warp,
                             uint32_t warps_per_cta);      /* fp8/src/lib.rs:203 */
void omega_gpu_fp8_set_cta_budget(uint32_t ctas);          /* fp8/src/lib.rs:204 */
/* fp8/src/lib.rs:729-750: 0 off; 1 scale dropped; 2 scale block never advances; 3 group table
 * entry skewed (TEST ONLY: deliberately wrong results a parity test must catch) */
void omega_gpu_fp8_test_set_mutant(int mutant);            /* fp8/src/lib.rs:205 */
void omega_gpu_fp8_test_set_no_fold(int on);               /* fp8/src/lib.rs:206 */

/* ================================================================== MoE router
 * crates/aien-omega-router/src/lib.rs:16-28 (contract), :78-132 (declarations) */
#define OMEGA_ROUTER_EXPERTS 128
#define OMEGA_ROUTER_HIDDEN 2048
#define OMEGA_ROUTER_TOPK 8
#define OMEGA_GPU_ROUTER_MAX_LAYERS 64

typedef struct OmegaGpuRouter OmegaGpuRouter;

/* router/src/lib.rs:49-65, layout asserted at :494-508 */
typedef struct OmegaGpuRouterInfo {
    uint32_t layer, warps, depth, threads;
    uint64_t weight_bytes;
    uint64_t elapsed_ns;
    uint64_t call_ns;
    uint32_t completion_marker;
    int32_t kernel_cache_hit;
} OmegaGpuRouterInfo;

/* router/src/lib.rs:85-90: experts 128 or 256, shared 0 or 1, 1 <= layers <= 64 */
int omega_gpu_router_alloc_shape(uint32_t layers, uint32_t experts, uint32_t shared,
                                 OmegaGpuRouter **out);
void omega_gpu_router_free(OmegaGpuRouter *r);                                 /* :91 */
/* :92-97: gate bf16 [experts + shared][2048], post_attention_layernorm weight f32 [2048] */
int omega_gpu_router_set_layer(OmegaGpuRouter *r, uint32_t layer, const uint16_t *gate_bf16,
                               const float *norm_w);
/* :98-103: {w_va, s_va} per expert (+ shared) of the gate|up and down FP8 tensors */
int omega_gpu_router_set_directory(OmegaGpuRouter *r, uint32_t layer, const uint64_t *gu,
                                   const uint64_t *dn);
/* :104-114: RMSNorm, logits, softmax, top-8 (descending logit, ties to the lower id),
 * renormalised when norm_topk; ids/weights to the host, x' * out_scale and both group tables to
 * the device */
int omega_gpu_router(OmegaGpuRouter *r, uint32_t layer, const float *x, float eps, int norm_topk,
                     float out_scale, uint32_t *ids, float *weights, OmegaGpuRouterInfo *info);
/* :115-120: addresses fixed for the router's life */
void omega_gpu_router_device_outputs(const OmegaGpuRouter *r, uint64_t *xout_va,
                                     uint64_t *tab_gu_va, uint64_t *tab_dn_va);
/* :121-126: any pointer may be NULL */
int omega_gpu_router_read_back(OmegaGpuRouter *r, float *xout, uint64_t *tab_gu,
                               uint64_t *tab_dn);
const char *omega_gpu_router_last_error(void);             /* :127 */
const char *omega_gpu_router_rc_name(int rc);              /* :128 */
/* :461-473: 0 off; 1 RMSNorm without the weight; 2 argmax mask removes id^1; 3 directory entry
 * of id^1 copied; 4 weights not normalised (TEST ONLY) */
void omega_gpu_router_test_set_mutant(int mutant);         /* :129 */

/* ================================================================== fused decode attention
 * crates/aien-omega-dattn/src/lib.rs:16-29 (contract), :80-136 (declarations) */
#define OMEGA_GPU_DATTN_Q_HEADS 32
#define OMEGA_GPU_DATTN_KV_HEADS 4
#define OMEGA_GPU_DATTN_HEAD_DIM 128
#define OMEGA_GPU_DATTN_QKV_WORDS 5120
#define OMEGA_DATTN_CHUNK 256
#define OMEGA_GPU_DATTN_MAX_POS 131072
#define OMEGA_GPU_DATTN_MAX_LAYERS 64

typedef struct OmegaGpuDecodeAttnCache OmegaGpuDecodeAttnCache;

/* dattn/src/lib.rs:57-75, layout asserted at :445-456 */
typedef struct OmegaGpuDecodeAttnInfo {
    uint32_t layer, pos, splits, per_split, depth, grid_x, grid_y, threads;
    uint64_t kv_bytes;
    uint64_t elapsed_ns;
    uint64_t call_ns;
    uint32_t completion_marker;
    int32_t kernel_cache_hit;
} OmegaGpuDecodeAttnInfo;

/* dattn/src/lib.rs:87-92: max_pos a multiple of 256 up to 131072, 1 <= layers <= 64 */
int omega_gpu_decode_attn_cache_alloc(uint32_t layers, uint32_t max_pos, double rope_theta,
                                      OmegaGpuDecodeAttnCache **out);
void omega_gpu_decode_attn_cache_free(OmegaGpuDecodeAttnCache *c);            /* :93 */
/* :94-99: per-head RMSNorm weights (128 f32 each) */
int omega_gpu_decode_attn_set_norms(OmegaGpuDecodeAttnCache *c, uint32_t layer,
                                    const float *q_norm, const float *k_norm);
/* :100-109: qkv = q[32][128] | k[4][128] | v[4][128] (pre-norm, pre-rope) -> out[32*128] *
 * out_scale; appends this position's K/V */
int omega_gpu_decode_attn(OmegaGpuDecodeAttnCache *c, uint32_t layer, uint32_t pos,
                          const float *qkv, float eps, float out_scale, float *out,
                          OmegaGpuDecodeAttnInfo *info);
const char *omega_gpu_decode_attn_last_error(void);       /* :110 */
const char *omega_gpu_decode_attn_rc_name(int rc);        /* :111 */
void omega_gpu_decode_attn_set_depth(uint32_t depth);     /* :112 */
void omega_gpu_decode_attn_set_per_split(uint32_t per_split); /* :113 */
/* :406-417: 0 off; 1 no RoPE; 2 V read one position late; 3 new K/V not written; 4 split
 * combine ignores the max; 9 (an extension) the in-launch split merge gives up at once, so the
 * call reports CHIP_FAIL with its message (TEST ONLY) */
void omega_gpu_decode_attn_test_set_mutant(int mutant);   /* :114 */
/* :117-125 and dattn/src/rows.rs:98-130: count consecutive bf16 K and V rows of (layer,kv_head) */
int omega_gpu_decode_attn_cache_write(OmegaGpuDecodeAttnCache *c, uint32_t layer,
                                      uint32_t kv_head, uint32_t pos, uint32_t count,
                                      const uint16_t *k_bf16, const uint16_t *v_bf16);
/* :126-133 and rows.rs:53-84 */
int omega_gpu_decode_attn_cache_read(OmegaGpuDecodeAttnCache *c, uint32_t layer, uint32_t kv_head,
                                     uint32_t pos, uint16_t *k_bf16, uint16_t *v_bf16);

/* ================================================================== bf16 streaming GEMV (lm_head)
 * crates/aien-omega-bf16/src/lib.rs:15-24 (contract), :70-101 (declarations) */
typedef struct OmegaGpuBf16Tensor OmegaGpuBf16Tensor;

/* bf16/src/lib.rs:43-60, layout asserted at :320-343 */
typedef struct OmegaGpuBf16Info {
    uint32_t n, k, rows_per_warp, warps_per_cta, depth, grid_x, steps;
    uint64_t weight_bytes;
    uint64_t elapsed_ns;
    uint64_t call_ns;
    uint32_t completion_marker;
    bool kernel_cache_hit;
    char target_chip[64];
    uint32_t sm_architecture;
} OmegaGpuBf16Info;

/* :78-83: [n][k] bf16, n >= 1, k % 256 == 0, 256 <= k <= 16384; NaN / inf refused */
int omega_gpu_bf16_tensor_upload(uint32_t n, uint32_t k, const uint16_t *w_bf16,
                                 OmegaGpuBf16Tensor **out);
void omega_gpu_bf16_tensor_free(OmegaGpuBf16Tensor *t);                       /* :84 */
/* :85-90: y = W x, deterministic summation order */
int omega_gpu_bf16_gemv_f32(const OmegaGpuBf16Tensor *t, const float *x, float *y,
                            OmegaGpuBf16Info *info);
/* :91-96 */
int omega_gpu_bf16_gemv_bf16(const OmegaGpuBf16Tensor *t, const uint16_t *x, float *y,
                             OmegaGpuBf16Info *info);
int omega_gpu_bf16_prepare(uint32_t k);                   /* :97 */
const char *omega_gpu_bf16_rc_name(int rc);               /* :98 */
const char *omega_gpu_bf16_last_error(void);              /* :99 */
void omega_gpu_bf16_test_set_mutant(int mutant);          /* :100 */

/* ================================================================== decode graph
 * crates/aien-omega-dgraph/src/lib.rs:16-30 (contract), :113-165 (declarations) */
#define OMEGA_GPU_DGRAPH_HIDDEN 2048
#define OMEGA_GPU_DGRAPH_MAX_LAYERS 64
#define OMEGA_GPU_DGRAPH_MAX_VOCAB (2048 * 2048)

typedef struct OmegaGpuDecodeGraph OmegaGpuDecodeGraph;

/* dgraph/src/lib.rs:83-93 (stats) and :95-105 (config), layouts asserted at :531-548 */
typedef struct OmegaGpuDecodeGraphStats {
    uint32_t launches;
    uint32_t submits;
    uint64_t chip_ns;
    uint64_t record_ns;
    uint64_t total_ns;
    uint32_t sems_done;
} OmegaGpuDecodeGraphStats;

typedef struct OmegaGpuDecodeGraphConfig {
    uint32_t layers;
    uint32_t vocab;
    float eps;
    int32_t norm_topk;
    void *router;        /* OmegaGpuRouter* */
    void *attn;          /* OmegaGpuDecodeAttnCache* */
    const void *lm_head; /* OmegaGpuBf16Tensor* */
} OmegaGpuDecodeGraphConfig;

/* launch kinds of the timeline (dgraph/src/lib.rs:47-61) */
enum {
    OMEGA_GPU_DGRAPH_K_NORM = 0, OMEGA_GPU_DGRAPH_K_QKV, OMEGA_GPU_DGRAPH_K_ATTN,
    OMEGA_GPU_DGRAPH_K_O_PROJ, OMEGA_GPU_DGRAPH_K_RES_ADD, OMEGA_GPU_DGRAPH_K_ROUTER,
    OMEGA_GPU_DGRAPH_K_GATE_UP, OMEGA_GPU_DGRAPH_K_SWIGLU, OMEGA_GPU_DGRAPH_K_DOWN,
    OMEGA_GPU_DGRAPH_K_COMBINE_NORM, OMEGA_GPU_DGRAPH_K_LM_HEAD, OMEGA_GPU_DGRAPH_K_ARGMAX
};

/* :121-124: the graph borrows the router, cache and lm_head handles; layers == 0 is refused
 * before any handle is read */
int omega_gpu_decode_graph_create(const OmegaGpuDecodeGraphConfig *cfg, OmegaGpuDecodeGraph **out);
void omega_gpu_decode_graph_free(OmegaGpuDecodeGraph *g);                      /* :125 */
/* :126-134: borrows the four FP8 tensors, copies input_norm f32 [2048] */
int omega_gpu_decode_graph_set_layer(OmegaGpuDecodeGraph *g, uint32_t layer, const void *qkv,
                                     const void *o, const void *gate_up, const void *down,
                                     const float *input_norm);
/* :135-138 */
int omega_gpu_decode_graph_set_final_norm(OmegaGpuDecodeGraph *g, const float *final_norm);
/* :139-145: one whole token as one submission -> the greedy token (lowest index of the max) */
int omega_gpu_decode_graph_token(OmegaGpuDecodeGraph *g, const float *x_embed, uint32_t pos,
                                 uint32_t *token, OmegaGpuDecodeGraphStats *st);
/* :146-151: any pointer may be NULL */
int omega_gpu_decode_graph_read(OmegaGpuDecodeGraph *g, float *x, float *hidden, float *logits);
/* :152: on = 1 submits and waits after every launch; 2 (an extension) launches the same kernels
 * directly without the graph and without waits */
void omega_gpu_decode_graph_set_flush_each(OmegaGpuDecodeGraph *g, int on);
/* :469-480: 0 off; 1 SwiGLU reads the wrong half; 2 combine skips expert 7; 3 attention written
 * at scale 2; extensions, on the chain form: 4 every routed expert e computed and reported as
 * (e + 1) % 128 (the engine's routing_mutant, qwen3_moe_omega.rs:3604-3608, a control of
 * own30b_check.rs:690-712); 5 the experts' FP8 block scales read as 1 (its scales-dropped
 * control, FP8 kernel mutant 1); on both forms: 9 every in-launch wait gives up at once
 * (TEST ONLY) */
void omega_gpu_decode_graph_test_set_mutant(OmegaGpuDecodeGraph *g, int mutant); /* :153 */
void omega_gpu_decode_graph_set_stamps(OmegaGpuDecodeGraph *g, int on);      /* :154 */
/* :155-160: launches + 1 GPU timestamps (ns) and one kind per launch; returns launches or rc<0 */
int omega_gpu_decode_graph_stamps(const OmegaGpuDecodeGraph *g, uint64_t *stamps, uint8_t *kinds,
                                  uint32_t cap);
const char *omega_gpu_decode_graph_kind_name(uint8_t kind);                  /* :161 */
const char *omega_gpu_session_last_error(void);                               /* :162 */

/* ================================================================== base ABI (omega_gpu.manifest)
 * crates/aien-omega-gpu/src/ffi.rs and abi/omega_gpu.manifest. The paged attention and the
 * pool allocation are implemented; the dense bf16 matmul / elementwise entries are outside the
 * decode step and answer BAD_ARGS (they exist so the archive qualifies against the manifest). */
#define OMEGA_GPU_MATMUL_OK 0
#define OMEGA_GPU_MATMUL_BAD_ARGS (-1)
#define OMEGA_GPU_MATMUL_TOO_LARGE (-2)
#define OMEGA_GPU_MATMUL_CODEGEN_FAIL (-3)
#define OMEGA_GPU_MATMUL_CHIP_FAIL (-4)
#define OMEGA_GPU_MATMUL_PARITY_FAIL (-5)
#define OMEGA_GPU_MATMUL_TILE_M 16
#define OMEGA_GPU_MATMUL_TILE_N 8
#define OMEGA_GPU_MATMUL_TILE_K 16
#define OMEGA_GPU_MATMUL_MAX_CTAS 1024
#define OMEGA_GPU_EW_OK 0
#define OMEGA_GPU_EW_BAD_ARGS (-1)
#define OMEGA_GPU_EW_TOO_LARGE (-2)
#define OMEGA_GPU_EW_CODEGEN_FAIL (-3)
#define OMEGA_GPU_EW_CHIP_FAIL (-4)
#define OMEGA_GPU_EW_UNWRITTEN (-5)
#define OMEGA_GPU_ATTN_OK 0
#define OMEGA_GPU_ATTN_BAD_ARGS (-1)
#define OMEGA_GPU_ATTN_TOO_LARGE (-2)
#define OMEGA_GPU_ATTN_CODEGEN_FAIL (-3)
#define OMEGA_GPU_ATTN_CHIP_FAIL (-4)
#define OMEGA_GPU_ATTN_UNWRITTEN (-5)
#define OMEGA_GPU_ATTN_KV_STAGED 0u
/* not in the reference manifest: KV read in place from device memory */
#define OMEGA_GPU_ATTN_KV_RESIDENT 1u

typedef struct OmegaGpuTensor OmegaGpuTensor;

/* ffi.rs:40-70 (manifest: 160 bytes) */
typedef struct OmegaGpuMatmulInfo {
    uint32_t m, k, n, padded_m, padded_n, k_slices, chip_calls, rows_per_call;
    uint64_t elapsed_ns;
    float max_abs_err, max_rel_err;
    size_t mismatch_count;
    bool parity_verified;
    uint32_t completion_marker;
    bool kernel_cache_hit;
    char target_chip[64];
    uint32_t sm_architecture;
    uint32_t grid_x, grid_y, padded_k;
    bool resident, oracle_ran;
    uint64_t call_ns;
} OmegaGpuMatmulInfo;

/* ffi.rs:107-118 (manifest: 40 bytes) */
typedef struct OmegaGpuAllocStats {
    uint64_t allocs, alloc_bytes, alloc_failures, frees, stale_refusals;
} OmegaGpuAllocStats;

/* ffi.rs:120-135 (manifest: 44 bytes) */
typedef struct OmegaGpuServingBounds {
    uint32_t max_context, max_seqs, num_q_heads, num_kv_heads, head_dim, kv_block_size, max_rows,
        max_k, max_n, max_n_one_row, kernel_slots;
} OmegaGpuServingBounds;

/* ffi.rs:218-235 (manifest: 120 bytes) */
typedef struct OmegaGpuEwInfo {
    uint32_t chip_calls;
    uint64_t elapsed_ns;
    uint32_t completion_marker, unwritten_words;
    bool kernel_cache_hit;
    uint32_t gpr_count, insn_count, threads_per_cta, ctas_last_launch;
    char target_chip[64];
    uint32_t sm_architecture;
    uint64_t call_ns;
} OmegaGpuEwInfo;

/* ffi.rs:306-338 (manifest: 176 bytes) */
typedef struct OmegaGpuAttnInfo {
    uint32_t chip_calls;
    uint64_t elapsed_ns;
    uint64_t call_ns;
    uint32_t completion_marker, unwritten_words, gpr_count, insn_count;
    bool kernel_cache_hit;
    uint32_t ctas_last_launch, threads_per_cta;
    char target_chip[64];
    uint32_t sm_architecture;
    uint64_t kv_bytes_staged, kv_bytes_naive;
    uint32_t kv_blocks_logical, kv_blocks_unique;
    uint64_t q_bytes, tab_bytes, out_bytes;
    uint32_t kv_source;
} OmegaGpuAttnInfo;

/* ffi.rs:385-400 = aien-kv-cache KvLayoutDesc (crates/aien-kv-cache/src/lib.rs:211-224) */
typedef struct OmegaGpuKvLayout {
    uint64_t block_stride_bytes, layer_stride_bytes, kv_plane_stride_bytes, token_stride_bytes,
        head_stride_bytes, pool_bytes;
    uint32_t num_blocks, num_layers, block_size;
} OmegaGpuKvLayout;

/* ffi.rs:137-214 (dense matmul family: stubs answering BAD_ARGS) */
int omega_gpu_matmul_bf16(uint32_t m, uint32_t k, uint32_t n, const uint16_t *a, const uint16_t *b,
                          float *c, OmegaGpuMatmulInfo *info);
int omega_gpu_matmul_f32(uint32_t m, uint32_t k, uint32_t n, const float *a, const float *b,
                         float *c, OmegaGpuMatmulInfo *info);
const char *omega_gpu_matmul_rc_name(int rc);
void omega_gpu_matmul_cache_clear(void);
int omega_gpu_tensor_upload_bf16(uint32_t k, uint32_t n, const uint16_t *b, OmegaGpuTensor **out);
int omega_gpu_tensor_upload_f32(uint32_t k, uint32_t n, const float *b, OmegaGpuTensor **out);
void omega_gpu_tensor_free(OmegaGpuTensor *t);
void omega_gpu_tensor_shape(const OmegaGpuTensor *t, uint32_t *k, uint32_t *n);
int omega_gpu_matmul_resident_bf16(uint32_t m, const uint16_t *a, const OmegaGpuTensor *b,
                                   float *c, OmegaGpuMatmulInfo *info);
int omega_gpu_matmul_resident_f32(uint32_t m, const float *a, const OmegaGpuTensor *b, float *c,
                                  OmegaGpuMatmulInfo *info);
const char *omega_gpu_matmul_last_error(void);
int omega_gpu_matmul_is_blocked(void);
void omega_gpu_device_close(void);
void omega_gpu_matmul_set_cta_budget(uint32_t ctas);
uint32_t omega_gpu_matmul_cta_budget(void);
/* ffi.rs:193-196: process-wide completion spin window (accepted and reported; HIP waits on
 * the stream) */
int omega_gpu_session_set_spin_us(uint32_t us);
uint32_t omega_gpu_session_spin_us(void);
int omega_gpu_reserve_serving(const OmegaGpuServingBounds *b);                /* ffi.rs:200 */
void omega_gpu_serving_release(void);                                         /* ffi.rs:201 */
int omega_gpu_matmul_prepare(uint32_t m, uint32_t k, uint32_t n);             /* ffi.rs:204 */
void omega_gpu_serving_seal(void);                                            /* ffi.rs:205 */
void omega_gpu_session_alloc_stats(OmegaGpuAllocStats *out);                  /* ffi.rs:207 */
/* ffi.rs:255-295 (elementwise family: stubs answering BAD_ARGS) */
int omega_gpu_rmsnorm_f32(uint32_t rows, uint32_t dim, const float *x, const float *weight,
                          float eps, float *out, OmegaGpuEwInfo *info);
int omega_gpu_rope_f32(uint32_t heads, uint32_t head_dim, const float *v, const float *cos_half,
                       const float *sin_half, float *out, OmegaGpuEwInfo *info);
int omega_gpu_swiglu_f32(uint32_t n, const float *gate, const float *up, float *out,
                         OmegaGpuEwInfo *info);
const char *omega_gpu_elementwise_rc_name(int rc);
/* ffi.rs:404-431 (dense f32 attention: stubs answering BAD_ARGS) */
int omega_gpu_gqa_attention_f32(const float *q, const float *k_cache, const float *v_cache,
                                uint32_t seq_len, uint32_t num_q_heads, uint32_t num_kv_heads,
                                uint32_t head_dim, float *out, OmegaGpuAttnInfo *info);
int omega_gpu_gqa_attention_rows_f32(const float *q, const float *k_cache, const float *v_cache,
                                     uint32_t base_len, uint32_t num_rows, uint32_t num_q_heads,
                                     uint32_t num_kv_heads, uint32_t head_dim, float *out,
                                     OmegaGpuAttnInfo *info);
/* ffi.rs:432-433: a KV pool the host writes and the GPU reads in place (pinned, device-mapped
 * host memory); one pool per process */
int omega_gpu_attention_pool_alloc(size_t bytes, void **cpu);
void omega_gpu_attention_pool_free(void);
/* ffi.rs:434-447: decode attention over the bf16 page pool of one sequence. q/out
 * [num_q_heads][head_dim] f32; block_ids lists the sequence's pages in token order. The pool may
 * be host memory (the referenced pages are staged) or device memory (read in place). */
int omega_gpu_paged_attention_bf16(const float *q, const void *pool, const OmegaGpuKvLayout *layout,
                                   const uint32_t *block_ids, uint32_t num_block_ids,
                                   uint32_t context_len, uint32_t layer_idx, uint32_t num_q_heads,
                                   uint32_t num_kv_heads, uint32_t head_dim, float *out,
                                   OmegaGpuAttnInfo *info);
/* The form of the paged calls (not in the reference ABI). on = 1 (the default): where a call's
 * split workgroups fit the device at once and its stream is not being captured into a graph,
 * the splits are merged inside the same launch (one launch per call); on = 0: always the split
 * launch and a combine launch. Both give the same results to f32 rounding. A merge whose bounded
 * wait runs out (test mutant 9 of omega_gpu_decode_attn_test_set_mutant makes it give up at
 * once) is reported as CHIP_FAIL by the host-buffer entries; the device-pointer entries return
 * before the work ends and write that call's merged heads as NaN. */
void omega_gpu_paged_attention_set_folded(int on);
/* ffi.rs:448-462: batched; block_tables [num_seqs][max_blocks_per_seq] (negative = none),
 * context_lens [num_seqs]; q/out [num_seqs][num_q_heads][head_dim] */
int omega_gpu_paged_attention_batch_bf16(const float *q, const void *pool,
                                         const OmegaGpuKvLayout *layout,
                                         const int32_t *block_tables, const int32_t *context_lens,
                                         uint32_t max_blocks_per_seq, uint32_t num_seqs,
                                         uint32_t layer_idx, uint32_t num_q_heads,
                                         uint32_t num_kv_heads, uint32_t head_dim, float *out,
                                         OmegaGpuAttnInfo *info);
const char *omega_gpu_attention_rc_name(int rc);                              /* ffi.rs:463 */
const char *omega_gpu_attention_last_error(void);                             /* ffi.rs:464 */

/* ================================================================== whole-prompt prefill
 * crates/aien-omega-pf/src/lib.rs:384-456 (the quantiser, the grouped W8A8 GEMM over a tile
 * table, the session buffers, the router logits and the MoE combine of the whole-prompt driver
 * qwen3_moe_omega_prefill.rs) and :542-571 (the prefill attention on the fused decode cache).
 * Every call is synchronous and returns the chip nanoseconds of its launches in *ns (NULL
 * allowed). Errors: omega_gpu_pf_rc_name + omega_gpu_session_last_error; the attention reports
 * through the decode attention family (omega_gpu_decode_attn_rc_name / _last_error). */
#define OMEGA_GPU_PF_PLAIN 0       /* y f32 rows of n */
#define OMEGA_GPU_PF_SWIGLU_NAT 2  /* tensor [E][2I][k] gate rows then up rows; y bf16 act rows of n / 2 */
#define OMEGA_QG_IN_F32 0
#define OMEGA_QG_IN_BF16 1
#define OMEGA_QG_TILE_BYTES 32
/* lib.rs:337-347: a session buffer (kind 0 device, 1 host-visible; cpu is the host view) */
typedef struct OmegaGpuMem {
    uint32_t handle_index, handle_generation, kind;
    void *cpu;
    uint64_t va, size;
} OmegaGpuMem;
/* lib.rs:83-93: one tile of the grouped GEMM: up to qgemm_bm() rows of one expert */
typedef struct OmegaGpuPfTile {
    uint64_t w_va, s_va;
    uint32_t row0, cnt;
    uint64_t pad;
} OmegaGpuPfTile;
/* lib.rs:362-376. Here chunks counts the call's work items, (tile of consecutive query tokens: 4
 * from a context of 1024 on, else 1; chunk of 32 pages) pairs, and grid_x = 4 kv heads x chunks */
typedef struct OmegaGpuPrefillAttnInfo {
    uint32_t layer, pos0, m, chunks, grid_x, grid_y, threads, splits, per_split;
    uint64_t elapsed_ns, call_ns;
    int32_t kernel_cache_hit;
} OmegaGpuPrefillAttnInfo;
const char *omega_gpu_pf_rc_name(int rc);                                              /* :385 */
int omega_gpu_pf_alloc_dev(size_t bytes, OmegaGpuMem *out);                            /* :387 */
int omega_gpu_pf_alloc_host(size_t bytes, OmegaGpuMem *out);                           /* :388 */
void omega_gpu_pf_free(OmegaGpuMem *m);                                                /* :389 */
int omega_gpu_pf_copy_va(uint64_t dst_va, uint64_t src_va, size_t bytes);             /* :390 */
void omega_gpu_pf_stats(uint64_t *chip_ns, uint64_t *launches);                        /* :391 */
void omega_gpu_pf_stats_reset(void);                                                   /* :392 */
/* :393-401: rows x k values (f32 or bf16) -> e4m3 codes [rows][k] and power-of-two block scales
 * f32 [rows][k / 128], the fake_quant rule (qwen3_moe_omega_prefill/fake_quant.rs:31-104) */
int omega_gpu_pf_quant(uint32_t k, uint32_t in_type, uint32_t rows, uint64_t x_va, uint64_t q_va, uint64_t s_va,
                       uint64_t *ns);
uint32_t omega_gpu_pf_qgemm_bm(void);                                                  /* :402 */
/* :403-410: the tile table of rows grouped by expert (lib.rs:122-160); returns the tile count,
 * 0 when it would exceed max */
uint32_t omega_gpu_pf_qgemm_tiles_va(uint32_t experts, const uint64_t *w_va, const uint64_t *s_va,
                                     const uint32_t *counts, void *tab, uint32_t max);
/* :411-424: for every tile, output rows row0 .. row0 + cnt of W_expert x dequant(activation row
 * rowidx[row] (or row when rowidx_va is 0)); the kernel reads activation rows (and row indices)
 * up to row0 + bm - 1 of every tile */
int omega_gpu_pf_qgemm(uint32_t n, uint32_t k, uint32_t layout, uint64_t tiles_va, uint32_t ntiles,
                       uint64_t rowidx_va, uint64_t xq_va, uint64_t xs_va, uint64_t y_va, uint64_t *ns);
uint32_t omega_gpu_pf_router_rows(void);                                               /* :430 */
void omega_gpu_pf_router_pack(uint32_t e, uint32_t k, const float *w, float *wq);      /* :431 */
/* :432-440: logits [rows][e] = the sequential f32 sum from -0.0 of w[ex][j] x[r][j] over the
 * packed weights (router_logits_ref, lib.rs:505-517); reads and writes whole tiles of
 * router_rows() rows */
int omega_gpu_pf_router_logits(uint32_t k, uint32_t e, uint32_t rows, uint64_t x_va, uint64_t wq_va,
                               uint64_t logits_va, uint64_t *ns);
/* :441-450: out[r] = sum over slots from +0.0 of wt[r][slot] * down[inv[r][slot]]
 * (moe_combine_ref, lib.rs:519-539) */
int omega_gpu_pf_moe_combine(uint32_t h, uint32_t top_k, uint32_t rows, uint64_t down_va, uint64_t inv_va,
                             uint64_t wt_va, uint64_t out_va, uint64_t *ns);
/* :543-553: layer `layer` of the m tokens at pos0 .. pos0 + m - 1 (0 .. pos0 - 1 already cached):
 * qkv f32 [m][5120] raw projection rows; appends their K / V; out f32 [m][4096] x out_scale */
int omega_gpu_prefill_attn(OmegaGpuDecodeAttnCache *c, uint32_t layer, uint32_t pos0, uint32_t m, const float *qkv,
                           float eps, float out_scale, float *out, OmegaGpuPrefillAttnInfo *info);
/* :559-571: the same on device rows (16-byte aligned) */
int omega_gpu_prefill_attn_dev(OmegaGpuDecodeAttnCache *c, uint32_t layer, uint32_t pos0, uint32_t m,
                               uint64_t qkv_va, float eps, float out_scale, uint64_t out_va,
                               OmegaGpuPrefillAttnInfo *info);

/* ================================================================== device-resident extensions
 * Not in the reference ABI: entry points for callers whose inputs already live in HBM (the
 * benchmark and the parity tests at full size). Same kernels as the entries above. */

/* The MoE routing plan of the whole-prompt driver on the host (not in the reference ABI: the
 * reference driver builds it in Rust, MoeBatchPlan::from_logits, moe_plan.rs:86-171, restated
 * here): per token the top_k experts by f32 total order with ties to the lower id, weights
 * expf(l - max) / sum in f32 in slot order, then the stable counting sort of the token-major
 * assignments by expert. Outputs: topk_ids / topk_weights [tokens][top_k], counts [experts],
 * grouped_token and assignment_to_grouped [tokens * top_k], grouped_to_assignment (may be NULL).
 * A non-finite logit is refused with BAD_ARGS naming the token and expert. No device work. */
int omega_gpu_pf_moe_plan(uint32_t tokens, uint32_t experts, uint32_t top_k, const float *logits, uint32_t *topk_ids,
                          float *topk_weights, uint32_t *counts, uint32_t *grouped_token,
                          uint32_t *assignment_to_grouped, uint32_t *grouped_to_assignment);
/* Persistent KV park / restore of the fused decode cache (not in the reference ABI: the reference
 * builds the HostPagedPoolV1 payload row by row through omega_gpu_decode_attn_cache_read /
 * _write, qwen3_moe_omega_kvio.rs:102-160). The payload of positions start .. start + len (start
 * a multiple of 16, start + len <= max_pos) is ceil(len / 16) blocks of [layer][K | V][token]
 * [kv head][dim] bf16 (qwen3_moe_omega_kvio.rs:17-24), rows at or past len zero; payload_len gives
 * its size, and a buffer of any other size is refused. Export writes the payload (host memory,
 * or device memory for _dev); import refuses a payload whose padding rows are not zero before
 * writing anything, then writes positions start .. start + len - 1 only. Synchronous; *ns (may
 * be NULL) is the call's chip time including the copies. */
uint64_t omega_gpu_decode_attn_cache_payload_len(const OmegaGpuDecodeAttnCache *c, uint32_t len);
int omega_gpu_decode_attn_cache_export(OmegaGpuDecodeAttnCache *c, uint32_t start, uint32_t len, void *out,
                                       uint64_t out_bytes, uint64_t *ns);
int omega_gpu_decode_attn_cache_export_dev(OmegaGpuDecodeAttnCache *c, uint32_t start, uint32_t len, void *out_dev,
                                           uint64_t out_bytes, uint64_t *ns);
int omega_gpu_decode_attn_cache_import(OmegaGpuDecodeAttnCache *c, uint32_t start, uint32_t len, const void *bytes,
                                       uint64_t nbytes, uint64_t *ns);
int omega_gpu_decode_attn_cache_import_dev(OmegaGpuDecodeAttnCache *c, uint32_t start, uint32_t len,
                                           const void *bytes_dev, uint64_t nbytes, uint64_t *ns);

/* The whole-prompt driver's residual and RMSNorm on the device (not in the reference ABI, whose
 * driver does both on the host, qwen3_moe_omega_prefill.rs:590-660): per row of k, x += add when
 * add_va is not 0 (in place), then out = x * scale * w, scale = 1 / sqrt(mean(x^2) + eps) with
 * an f64 sum of squares rounded to f32 (tensor.rs:94-110). Synchronous; chip ns in *ns. */
int omega_gpu_pf_residual_norm(uint32_t k, uint32_t rows, uint64_t x_va, uint64_t add_va, uint64_t w_va, float eps,
                               uint64_t out_va, uint64_t *ns);
/* Synthetic random-init FP8 tensor generated on the device: W ~ N(0, sigma) per element from
 * the counter-based generator (seed, tensor_id, element index), per 128x128 block
 * s = bf16(absmax / 448), q = e4m3(W / s). Bit-identical to the CPU generator of the tests. */
int omega_gpu_fp8_tensor_synth(uint32_t experts, uint32_t n, uint32_t k, uint64_t seed,
                               uint64_t tensor_id, float sigma, OmegaGpuFp8Tensor **out);
/* bf16 [n][k] N(0, sigma) synthetic tensor on the device */
int omega_gpu_bf16_tensor_synth(uint32_t n, uint32_t k, uint64_t seed, uint64_t tensor_id,
                                float sigma, OmegaGpuBf16Tensor **out);
/* the same generator on the host: count bf16 values of N(0, sigma) (or 1 + N(0, sigma)) */
void omega_gpu_synth_bf16_host(uint64_t seed, uint64_t tensor_id, size_t count, float sigma,
                               int one_plus, uint16_t *out);
/* the same generator into a caller's device buffer: count bf16 values of N(0, sigma), enqueued
 * on the library's stream (no synchronisation) */
int omega_gpu_synth_bf16_dev(void *dst, uint64_t count, uint64_t seed, uint64_t tensor_id, float sigma);
/* device-pointer GEMV: x_dev f32[k], y_dev f32[n]; no host copies, no synchronisation
 * (stream = the library's stream) */
int omega_gpu_fp8_gemv_dev(const OmegaGpuFp8Tensor *t, uint32_t expert, const float *x_dev,
                           float *y_dev);
/* device-pointer batched paged attention over a device pool (the batched entry without staging
 * and host copies); all pointers are device addresses */
int omega_gpu_paged_attention_batch_dev(const float *q_dev, const void *pool_dev,
                                        const OmegaGpuKvLayout *layout,
                                        const int32_t *block_tables_dev,
                                        const int32_t *context_lens_dev,
                                        uint32_t max_blocks_per_seq, uint32_t num_seqs,
                                        uint32_t max_context, uint32_t layer_idx,
                                        uint32_t num_q_heads, uint32_t num_kv_heads,
                                        uint32_t head_dim, float *out_dev);
/* No counterpart in the reference: omega_gpu_paged_attention_batch_dev for callers that cannot
 * allocate device memory (code under HIP graph capture, fixed serving loops, harnesses that forbid
 * hipMalloc). Same arguments, kernels and results; the split partials live in a static device
 * array of 16 MiB (per GPU, held until the process ends) instead of the library's growable
 * scratch, and the call makes no hipMalloc / hipFree. A shape whose partials exceed it
 * (num_seqs x num_q_heads x splits x 528 bytes) is refused with OMEGA_GPU_ATTN_TOO_LARGE before
 * any device work. Every call on one GPU shares the array: calls run in order on the library's
 * stream, but a replay of a graph holding this call that overlaps another such call on the same
 * GPU races on it. */
int omega_gpu_paged_attention_batch_dev_noalloc(const float *q_dev, const void *pool_dev,
                                                const OmegaGpuKvLayout *layout,
                                                const int32_t *block_tables_dev,
                                                const int32_t *context_lens_dev,
                                                uint32_t max_blocks_per_seq, uint32_t num_seqs,
                                                uint32_t max_context, uint32_t layer_idx,
                                                uint32_t num_q_heads, uint32_t num_kv_heads,
                                                uint32_t head_dim, float *out_dev);
/* The batched serving step's attention on its own (not in the reference ABI; the ragged batch of
 * paged_attention_batch_bf16, crates/aien-omega-gpu/src/lib.rs:910-1041, with GQA 32 q / 4 kv
 * heads of 128 over 16-token pages): sequence s attends over positions 0..=positions[s] (host
 * array) through its table row; the pages of all sequences are split into equal runs per
 * wavefront (the work plan of omega_gpu_batch_decode_step). q_dev [num_seqs][32][128] f32
 * (post-norm, post-RoPE), out_dev [num_seqs][32][128] f32; num_seqs <= 32. Synchronises the
 * library stream before returning. */
int omega_gpu_paged_attention_items_dev(const float *q_dev, const void *pool_dev, const OmegaGpuKvLayout *layout,
                                        const int32_t *block_tables_dev, uint32_t max_blocks_per_seq,
                                        const uint32_t *positions, uint32_t num_seqs, uint32_t layer_idx,
                                        float *out_dev);
/* the decode graph with the embedding row gathered on the device: set a [vocab][2048] bf16
 * tensor once, then each token passes only its id */
int omega_gpu_decode_graph_set_embedding(OmegaGpuDecodeGraph *g, const void *embed_bf16);
int omega_gpu_decode_graph_token_id(OmegaGpuDecodeGraph *g, uint32_t token_in, uint32_t pos,
                                    uint32_t *token, OmegaGpuDecodeGraphStats *st);
/* the routed expert ids and weights of every layer of the decode graph's last token
 * ([layers][8] each; either pointer may be NULL) — a trace for parity checks */
int omega_gpu_decode_graph_read_routes(OmegaGpuDecodeGraph *g, uint32_t *ids, float *weights);
/* with stamps on, the per-launch times (ns) of the last token: replaying the graph, the span
 * between the event-record nodes around each launch (its share of the replayed token, launch gap
 * included); with flush_each (direct launches), start to end of each dispatch as the hardware
 * recorded it (no launch gaps). Returns launches or rc<0 */
int omega_gpu_decode_graph_kernel_ns(const OmegaGpuDecodeGraph *g, uint64_t *ns, uint32_t cap);
/* Teacher forcing for parity tests (not in the reference ABI): ids [layers][8] expert ids
 * (< 128) used by the following tokens in place of each layer's top-8 ranking, in slot order,
 * their weights the softmax of the device's own router logits over that set; a layer whose row
 * starts with OMEGA_GPU_DGRAPH_RANK (0xFFFFFFFF; the rest of the row ignored) ranks its own
 * logits as usual; NULL turns the forcing off. Lets a full-size decode be compared with the
 * oracle past a routing near-tie. */
#define OMEGA_GPU_DGRAPH_RANK 0xFFFFFFFFu
int omega_gpu_decode_graph_test_force_routes(OmegaGpuDecodeGraph *g, const uint32_t *ids);
/* Layer trace for parity tests (not in the reference ABI; the engine's trace_layers and
 * LayerTrace, qwen3_moe_omega.rs:3227-3243, read by own30b_check.rs:632-700): with n layers
 * (<= 8, distinct) every following token runs the chain form as direct launches and records, per
 * traced layer, the residual row entering it, the o projection's output, the residual after the
 * attention (x'), the router's normed row, the routed ids and weights in slot order, the MoE
 * output (the slot-order combine, no residual) and the residual leaving it. n = 0 turns the trace
 * off. read_trace copies the last token's record of the i-th traced layer; any pointer may be
 * NULL ([2048] floats each, ids and weights [8]). */
int omega_gpu_decode_graph_test_set_trace(OmegaGpuDecodeGraph *g, const uint32_t *layers, uint32_t n);
int omega_gpu_decode_graph_test_read_trace(OmegaGpuDecodeGraph *g, uint32_t i, float *x_in,
                                           float *attn_proj, float *x_mid, float *post,
                                           uint32_t *experts, float *weights, float *moe_out,
                                           float *x_out);
/* The decode graph's form (not in the reference ABI; the one-submission contract of
 * crates/aien-omega-dgraph/src/lib.rs:16-30 holds either way). on = 0 (the default): the chain of
 * six launches per layer; on = 1, where the device holds all 256 workgroups at once: each token's
 * graph is one persistent launch of every layer plus the lm_head launch. Both compute every value
 * the same way and give the same bits. Stamps run the chain; flush_each 3 runs the persistent
 * form as direct launches. Returns the form in use after the call: 1 persistent, 0 chain. */
int omega_gpu_decode_graph_set_persistent(OmegaGpuDecodeGraph *g, int on);
/* Stage stamps of the persistent form (not in the reference ABI): with on, each token records
 * on the GPU's constant clock, per layer, the end of its 5 stages — input row in every
 * workgroup, attention row, residual after the attention, route inputs (logits and x'), down
 * rows — as ns since the launch started. stage_ns copies the last token's layers * 5 values
 * into ns; returns their count or rc < 0 (BAD_ARGS when the last token kept none). */
void omega_gpu_decode_graph_set_stage_stamps(OmegaGpuDecodeGraph *g, int on);
int omega_gpu_decode_graph_stage_ns(const OmegaGpuDecodeGraph *g, uint64_t *ns, uint32_t cap);
/* Batched MoE block (not in the reference ABI; the expert FFN of a decode step at token batch
 * T <= 64, the reference's per-token FP8 arm qwen3_moe_omega.rs:4287-4318 batched): for each of
 * `tokens` rows of h [T][2048] f32, RMSNorm with the router's layer weights, router logits, top-8
 * (ids and weights bit-exact with the per-token route), then gate|up, SwiGLU and down of the
 * routed experts grouped by expert on the FP8 matrix cores, combined in slot order:
 * moe_out [T][2048] (no residual). Errors are reported by omega_gpu_fp8gemm_last_error. */
int omega_gpu_moe_batch_f32(const OmegaGpuRouter *router, uint32_t layer, const OmegaGpuFp8Tensor *gate_up,
                            const OmegaGpuFp8Tensor *down, uint32_t tokens, const float *h, float eps,
                            int norm_topk, uint32_t *ids, float *weights, float *moe_out);
/* the same on device pointers, enqueued on the library's stream; out = resid + moe when resid_dev
 * is not NULL (resid_dev may equal out_dev). It returns before the work completes, so a grouping
 * planner whose bounded wait runs out is not reported here: the block then adds no expert rows
 * (out = resid, or 0 without resid) and the ids / weights are the rankings' own. The f32 entry
 * and the batched decode step report that case as CHIP_FAIL. */
int omega_gpu_moe_batch_dev(const OmegaGpuRouter *router, uint32_t layer, const OmegaGpuFp8Tensor *gate_up,
                            const OmegaGpuFp8Tensor *down, uint32_t tokens, const float *h_dev, float eps,
                            int norm_topk, const float *resid_dev, uint32_t *ids_dev, float *weights_dev,
                            float *out_dev);
/* test mutants of the batched MoE block: 1 rank mask on id^1, 2 weights not normalised, 5 gate and
 * up swapped, 6 slot 7 dropped from the combine, 7 one activation term (a plain fp8 cast), 9 the
 * grouping planner's wait (more than 4 tokens) gives up at once (TEST ONLY) */
void omega_gpu_moe_test_set_mutant(int mutant);
/* Batched serving decode (not in the reference ABI; the multi-sequence decode that
 * crates/aien-serve-http's Engine::concurrency / generate_group would drive for the 30B,
 * engine.rs:131-179): one greedy step of up to 32 sequences of the Qwen3-30B-A3B FP8 model
 * (the per-token semantics of Qwen3MoeOmegaEngine::step, qwen3_moe_omega.rs:4096-4345) over
 * the caller's device KV pool in the aien-kv-cache page layout (crates/aien-kv-cache/src/
 * lib.rs:129-365), read and written in place. Each step appends every sequence's K/V at its
 * position through its page table and attends over positions 0..=pos. One hipGraph per batch
 * size; errors are reported by omega_gpu_session_last_error. The router, tensors, pool and
 * page tables are borrowed and must outlive the handle. */
typedef struct OmegaGpuBatchDecode OmegaGpuBatchDecode;
typedef struct OmegaGpuBatchDecodeConfig {
    uint32_t layers, vocab, max_seqs, max_blocks_per_seq, max_pos;
    float eps;
    int32_t norm_topk;
    double rope_theta;
    void *router;    /* OmegaGpuRouter (128 experts; the post-attention norm per layer) */
    void *lm_head;   /* OmegaGpuBf16Tensor [vocab][2048], vocab a multiple of 16 */
    void *embed;     /* OmegaGpuBf16Tensor [vocab][2048] */
    void *pool;      /* device KV pool */
    OmegaGpuKvLayout layout;
} OmegaGpuBatchDecodeConfig;
int omega_gpu_batch_decode_create(const OmegaGpuBatchDecodeConfig *cfg, OmegaGpuBatchDecode **out);
void omega_gpu_batch_decode_free(OmegaGpuBatchDecode *b);
/* q|k|v 1x5120x2048, o 1x2048x4096, gate|up 128x1536x2048, down 128x2048x768 FP8 tensors, the
 * input norm [2048] and the q / k head norms [128] of a layer */
int omega_gpu_batch_decode_set_layer(OmegaGpuBatchDecode *b, uint32_t layer, const void *qkv, const void *o,
                                     const void *gate_up, const void *down, const float *input_norm,
                                     const float *q_norm, const float *k_norm);
int omega_gpu_batch_decode_set_final_norm(OmegaGpuBatchDecode *b, const float *final_norm);
/* page tables [seqs][max_blocks_per_seq] (-1: none), copied to the device */
int omega_gpu_batch_decode_set_tables(OmegaGpuBatchDecode *b, uint32_t seqs, const int32_t *tables);
/* keep every step's logits [seqs][vocab] for omega_gpu_batch_decode_read (off by default) */
void omega_gpu_batch_decode_set_keep_logits(OmegaGpuBatchDecode *b, int on);
/* launch the step's kernels directly instead of replaying the hipGraph (profilers that cannot
 * follow graph capture); the same kernels and arguments */
void omega_gpu_batch_decode_set_eager(OmegaGpuBatchDecode *b, int on);
/* one step: sequence s feeds tokens[s] at positions[s]; next_tokens[s] = its greedy token */
int omega_gpu_batch_decode_step(OmegaGpuBatchDecode *b, uint32_t seqs, const uint32_t *tokens,
                                const uint32_t *positions, uint32_t *next_tokens);
/* the last step's residual rows x, final-normed rows, logits (kept) [seqs][...] and routed expert
 * ids [layers][seqs][8]; any pointer may be NULL */
int omega_gpu_batch_decode_read(OmegaGpuBatchDecode *b, uint32_t seqs, float *x, float *hidden, float *logits,
                                uint32_t *route_ids);
/* the library's HIP stream (hipStream_t) and a full synchronisation of it */
void *omega_gpu_stream(void);
int omega_gpu_sync(void);

#ifdef __cplusplus
}
#endif

/* layout checks for C++ and C11 consumers alike */
#if defined(__cplusplus) || (defined(__STDC_VERSION__) && __STDC_VERSION__ >= 201112L)
#ifndef __cplusplus
#include <assert.h>
#endif
static_assert(sizeof(OmegaGpuMem) == 40, "OmegaGpuMem");
static_assert(offsetof(OmegaGpuMem, va) == 24, "OmegaGpuMem.va");
static_assert(sizeof(OmegaGpuPfTile) == 32, "OMEGA_QG_TILE_BYTES");
static_assert(sizeof(OmegaGpuPrefillAttnInfo) == 64, "PrefillAttnInfo");
static_assert(offsetof(OmegaGpuPrefillAttnInfo, elapsed_ns) == 40, "PrefillAttnInfo.elapsed_ns");
static_assert(offsetof(OmegaGpuPrefillAttnInfo, kernel_cache_hit) == 56, "PrefillAttnInfo.hit");
static_assert(sizeof(OmegaGpuFp8Info) == 160, "Fp8Info");
static_assert(offsetof(OmegaGpuFp8Info, weight_bytes) == 48, "Fp8Info.weight_bytes");
static_assert(offsetof(OmegaGpuFp8Info, kernel_cache_hit) == 84, "Fp8Info.kernel_cache_hit");
static_assert(offsetof(OmegaGpuFp8Info, sm_architecture) == 152, "Fp8Info.sm_architecture");
static_assert(sizeof(OmegaGpuFp8GemmInfo) == 80, "GemmInfo");
static_assert(offsetof(OmegaGpuFp8GemmInfo, passes_max) == 36, "GemmInfo.passes_max");
static_assert(offsetof(OmegaGpuFp8GemmInfo, weight_bytes) == 40, "GemmInfo.weight_bytes");
static_assert(offsetof(OmegaGpuFp8GemmInfo, kernel_cache_hit) == 76, "GemmInfo.hit");
static_assert(sizeof(OmegaGpuRouterInfo) == 48, "RouterInfo");
static_assert(offsetof(OmegaGpuRouterInfo, kernel_cache_hit) == 44, "RouterInfo.hit");
static_assert(sizeof(OmegaGpuDecodeAttnInfo) == 64, "DecodeAttnInfo");
static_assert(offsetof(OmegaGpuDecodeAttnInfo, kv_bytes) == 32, "DecodeAttnInfo.kv_bytes");
static_assert(offsetof(OmegaGpuDecodeAttnInfo, kernel_cache_hit) == 60, "DecodeAttnInfo.hit");
static_assert(sizeof(OmegaGpuBf16Info) == 136, "Bf16Info");
static_assert(offsetof(OmegaGpuBf16Info, weight_bytes) == 32, "Bf16Info.weight_bytes");
static_assert(offsetof(OmegaGpuBf16Info, target_chip) == 61, "Bf16Info.target_chip");
static_assert(offsetof(OmegaGpuBf16Info, sm_architecture) == 128, "Bf16Info.sm_architecture");
static_assert(sizeof(OmegaGpuDecodeGraphConfig) == 40, "GraphConfig");
static_assert(offsetof(OmegaGpuDecodeGraphConfig, router) == 16, "GraphConfig.router");
static_assert(offsetof(OmegaGpuDecodeGraphConfig, lm_head) == 32, "GraphConfig.lm_head");
static_assert(sizeof(OmegaGpuDecodeGraphStats) == 40, "GraphStats");
static_assert(offsetof(OmegaGpuDecodeGraphStats, sems_done) == 32, "GraphStats.sems_done");
static_assert(sizeof(OmegaGpuMatmulInfo) == 160, "MatmulInfo");
static_assert(offsetof(OmegaGpuMatmulInfo, call_ns) == 152, "MatmulInfo.call_ns");
static_assert(sizeof(OmegaGpuAllocStats) == 40, "AllocStats");
static_assert(sizeof(OmegaGpuServingBounds) == 44, "ServingBounds");
static_assert(sizeof(OmegaGpuEwInfo) == 120, "EwInfo");
static_assert(offsetof(OmegaGpuEwInfo, call_ns) == 112, "EwInfo.call_ns");
static_assert(sizeof(OmegaGpuAttnInfo) == 176, "AttnInfo");
static_assert(offsetof(OmegaGpuAttnInfo, sm_architecture) == 116, "AttnInfo.sm_architecture");
static_assert(offsetof(OmegaGpuAttnInfo, kv_bytes_staged) == 120, "AttnInfo.kv_bytes_staged");
static_assert(offsetof(OmegaGpuAttnInfo, kv_blocks_logical) == 136, "AttnInfo.kv_blocks_logical");
static_assert(offsetof(OmegaGpuAttnInfo, q_bytes) == 144, "AttnInfo.q_bytes");
static_assert(offsetof(OmegaGpuAttnInfo, kv_source) == 168, "AttnInfo.kv_source");
static_assert(sizeof(OmegaGpuKvLayout) == 64, "KvLayout");
static_assert(sizeof(OmegaGpuBatchDecodeConfig) == 136, "BatchDecodeConfig");
static_assert(offsetof(OmegaGpuBatchDecodeConfig, layout) == 72, "BatchDecodeConfig.layout");
static_assert(offsetof(OmegaGpuKvLayout, block_size) == 56, "KvLayout.block_size");
#endif

#endif /* OMEGA_GPU_H */
