/*
 * CPU ORACLE — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's Rust host oracles for the Qwen3-30B-A3B FP8 decode
 * step (aien-dev/aien-sovereign-core-mv, paths relative to its repository root). Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and only as the
 * checker or the timed CPU baseline: the MI355X product path (libomega_gpu) never links it.
 *
 * Every function names the reference file:line it follows. Summation orders, the f32/f64 split
 * and the rounding rules are kept exactly as the Rust states them, so that on the same inputs the
 * results are bit-identical to the Rust code (IEEE f32/f64 without contraction; compiled with
 * -ffp-contract=off; expf/exp/sin/cos/pow/log2 from the same glibc libm the Rust std calls).
 *
 * Parity pins (see tests/test_oracle_*.py): every function below is checked against a golden
 * vector, a known-answer test held by the reference's own tests, or a closed form / brute force
 * chosen so that a dropped term, a wrong sign or index or a transposed operand fails.
 * One refinement is not in the reference and is marked as such: oref_router_logits_f64.
 */
#ifndef OMEGA_ORACLE_H
#define OMEGA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- codecs ---------------- */
float oref_bf16_to_f32(uint16_t bits);                 /* qwen3_moe.rs:481-483 */
uint16_t oref_f32_to_bf16(float v);                    /* qwen3_moe.rs:486-493 (NaN keeps NaN) */
uint16_t oref_kv_f32_to_bf16(float v);                 /* aien-kv-cache/src/lib.rs:116-121 */
float oref_e4m3_to_f32(uint8_t bits);                  /* qwen3_moe.rs:496-508 */
uint8_t oref_f32_to_e4m3(float v);                     /* qwen3_moe.rs:515-547 (binary search) */
uint8_t oref_f32_to_e4m3_fast(float v);                /* same rounding, bit arithmetic */
/* fake_quant.rs: the W8A8 activation quantiser */
uint8_t oref_e4m3_rne_sat(float f);                    /* fake_quant.rs:29-57 */
float oref_fq_e4m3_to_f32(uint8_t c);                  /* fake_quant.rs:60-72 */
void oref_block_scale(float m, float *scale, float *inv); /* fake_quant.rs:75-83 */
void oref_quant_row(const float *x, int k, uint8_t *q, float *s); /* fake_quant.rs:87-106 */
void oref_fake_quant_row(float *x, int k);             /* fake_quant.rs:109-117 */
void oref_bf16_round_row(float *x, int k);             /* fake_quant.rs:120-124 */
void oref_quantize_block128(float *x, int k);          /* qwen3_moe.rs:559-567 */

/* ---------------- generators ---------------- */
float oref_prand(uint64_t seed, uint64_t idx);         /* qwen3_moe_omega.rs:1654-1662 */
uint64_t oref_splitmix64(uint64_t x);
/* Counter-based approximately-normal value (12-uniform Irwin-Hall), identical on CPU and GPU:
 * z = (sum of twelve 16-bit uniforms - 393210) * (sigma * 2^-16). Not from the reference: the
 * reference's own fill (prand) is uniform; this generator gives the N(0, sigma) the benchmark
 * configurations ask for. */
float oref_synth_normal(uint64_t seed, uint64_t tensor, uint64_t idx, float sigma);
/* bf16 tensor of N(0, sigma) values (RNE), or of 1 + N(0, sigma) when `one_plus` */
void oref_synth_bf16(uint64_t seed, uint64_t tensor, size_t count, float sigma, int one_plus,
                     uint16_t *out);
void oref_synth_f32(uint64_t seed, uint64_t tensor, size_t count, float sigma, int one_plus,
                    float *out);
/* FP8 block-quantised [experts][n][k] tensor: W ~ N(0, sigma) per element, per 128x128 block
 * s = bf16(absmax / 448), q = e4m3(W / s) (RNE, saturating). */
void oref_synth_fp8(uint64_t seed, uint64_t tensor, int experts, int n, int k, float sigma,
                    uint8_t *w, uint16_t *scale_bf16);

/* ---------------- FP8 / bf16 GEMV ---------------- */
/* HostFp8::grouped_f32 (qwen3_moe_omega.rs:2114-2139): acc += e4m3(w) * bf16(s) * x, per row
 * in column order, f32. x is k values (x_rows = 1) or groups * k values. */
void oref_fp8_grouped(const uint8_t *w, const uint16_t *s, int experts, int n, int k, int groups,
                      const uint32_t *ids, const float *x, int x_rows, float *y);
/* dequant_matvec (qwen3_moe.rs:595-619): per 128 block dot, times scale, blocks summed */
void oref_dequant_matvec(const uint8_t *w, const uint16_t *s, int rows, int cols, const float *v,
                         float *out);
/* FakeLmHead::logits_f32 (qwen3_moe_omega.rs:2015-2028): y[r] = sum_c bf16(W[r][c]) * x[c] */
void oref_bf16_gemv(const uint16_t *w, int n, int k, const float *x, float *y);
void oref_bf16_gemv_mt(const uint16_t *w, int n, int k, const float *x, float *y, int threads);
void oref_fp8_grouped_mt(const uint8_t *w, const uint16_t *s, int experts, int n, int k,
                         int groups, const uint32_t *ids, const float *x, int x_rows, float *y,
                         int threads);
/* sample_argmax (tensor.rs:299-318): lowest index of the max (strict > scan) */
uint32_t oref_argmax(const float *logits, int n);

/* ---------------- norms, rope, attention ---------------- */
void oref_rmsnorm(const float *x, const float *w, int dim, float eps, float *out); /* tensor.rs:94-110 */
void oref_rmsnorm_per_head(const float *x, const float *w, float eps, int heads, int hd,
                           float *out);        /* qwen3_coder.rs:306-320 */
void oref_rope_cos_sin(double theta, int hd, int pos, float *cos_out, float *sin_out);
/* tensor.rs:150-161 with RopeParams::inv_freq (aien-abi-core/src/lib.rs:106-113) */
void oref_apply_rope(float *q, float *k, int pos, int qh, int kvh, int hd, double theta);
/* tensor.rs:164-190 */
/* scaled_dot_product_attention_single (tensor.rs:193-250). K, V: [ctx][kvh * hd] */
void oref_sdpa(const float *q, const float *k, const float *v, int ctx, int qh, int kvh, int hd,
               float *out);

/* ---------------- routing and MoE ---------------- */
/* router logits, f32 products summed in index order (qwen3_moe_omega.rs:1968-1976, 5637-5650) */
void oref_router_logits(const uint16_t *gate_bf16, const float *post, int experts, int hidden,
                        float *logits);
/* REFINEMENT (not in the reference): the same dot products accumulated in f64 and rounded once
 * to f32, so the value does not depend on the summation order (GPU and CPU agree). */
void oref_router_logits_f64(const uint16_t *gate_bf16, const float *post, int experts, int hidden,
                            float *logits);
/* MoeBatchPlan::from_logits (moe_plan.rs:86-171). Returns 0, or -1 for a bad shape, or
 * -(2 + token*experts + expert) for a non-finite logit. Any output pointer may be NULL except
 * topk_experts and topk_weights. */
int oref_moe_plan(const float *logits, int tokens, int experts, int top_k, uint32_t *topk_experts,
                  float *topk_weights, uint32_t *expert_offsets, uint32_t *grouped_to_assignment,
                  uint32_t *assignment_to_grouped, uint32_t *grouped_token_ids);
/* MoeBatchPlan::reduce_grouped (moe_plan.rs:213-233) */
void oref_reduce_grouped(const uint32_t *assignment_to_grouped, const float *topk_weights,
                         int tokens, int top_k, const float *grouped, int hidden, float *out);
/* swiglu (qwen3_moe_omega.rs:5616-5621): act[j] = g / (1 + exp(-g)) * u */
void oref_swiglu(const float *gu, int i, float *act);
/* FakeRouter::route (qwen3_moe_omega.rs:1943-1998): RMSNorm, logits, plan of one token.
 * refined != 0 uses oref_router_logits_f64. post and logits may be NULL. */
int oref_route(const uint16_t *gate_bf16, const float *norm_w, int experts, int hidden, int top_k,
               const float *x, float eps, int refined, uint32_t *ids, float *weights, float *post,
               float *logits);
/* reference_moe_forward_with (qwen3_moe.rs:626-686), one token per row; quantize != 0 is
 * OracleActivations::Fp8Block128. gate_up [E][2i][h], down [E][h][i]. */
void oref_moe_forward(const uint8_t *gu_w, const uint16_t *gu_s, const uint8_t *dn_w,
                      const uint16_t *dn_s, int hidden, int inter, int tokens, int top_k,
                      const uint32_t *topk_experts, const float *topk_weights, const float *x,
                      int quantize, float *out);
/* Engine step MoE block for one token (qwen3_moe_omega.rs:4287-4318): gate|up grouped GEMV on
 * the post row, SwiGLU per slot, down grouped GEMV with a row per slot, combine in slot order
 * from zero. out = moe_out (the residual add is the caller's). w8a8 != 0 applies the W8A8
 * control's activation rounding (w8a8_control.rs:21-25, 161-171). */
void oref_moe_block(const uint8_t *gu_w, const uint16_t *gu_s, const uint8_t *dn_w,
                    const uint16_t *dn_s, int experts, int hidden, int inter, int top_k,
                    const uint32_t *ids, const float *weights, const float *post, int w8a8,
                    float *moe_out);

/* ---------------- KV page layout (aien-kv-cache/src/lib.rs:211-347) ---------------- */
typedef struct {
    uint64_t block_stride_bytes, layer_stride_bytes, kv_plane_stride_bytes, token_stride_bytes,
        head_stride_bytes, pool_bytes;
    uint32_t num_blocks, num_layers, block_size;
} oref_kv_layout;
void oref_kv_layout_bf16(uint32_t num_blocks, uint32_t block_size, uint32_t layers,
                         uint32_t kv_heads, uint32_t head_dim, oref_kv_layout *out);
uint64_t oref_kv_element_offset(const oref_kv_layout *l, uint32_t block, uint32_t layer,
                                int is_value, uint32_t token, uint32_t head, uint32_t dim);
/* write_token_kv, bf16 arm (lib.rs:586-622) */
void oref_kv_write_token(uint8_t *pool, const oref_kv_layout *l, uint32_t block, uint32_t layer,
                         uint32_t token, int kv_dim, const float *k, const float *v);
/* read_token_kv, bf16 arm (lib.rs:624-659) */
void oref_kv_read_token(const uint8_t *pool, const oref_kv_layout *l, uint32_t block,
                        uint32_t layer, uint32_t token, int kv_dim, float *k, float *v);
/* paged decode attention of one sequence: gather_layer_kv (lib.rs:661-691) then sdpa */
void oref_paged_attention(const float *q, const uint8_t *pool, const oref_kv_layout *l,
                          const int32_t *block_table, int context_len, int layer, int qh, int kvh,
                          int hd, float *out);
uint64_t oref_fnv1a64(const uint8_t *bytes, size_t n);

/* ---------------- fused decode attention cache (aien-omega-dattn) ---------------- */
/* The cache keeps bf16 rows (kv_head, pos) per layer and plane, as the dattn row helpers
 * (dattn/src/rows.rs:18-24) describe. */
typedef struct oref_dattn oref_dattn;
oref_dattn *oref_dattn_alloc(int layers, int max_pos, double theta);
void oref_dattn_free(oref_dattn *c);
void oref_dattn_set_norms(oref_dattn *c, int layer, const float *q_norm, const float *k_norm);
/* One layer step (dattn/src/lib.rs:16-29): per-head RMSNorm of q and k, RoPE at pos, bf16 K/V
 * append at pos, f64 attention over 0..=pos (the HostPoolKv arm: bf16 K/V, f32 q,
 * qwen3_moe_omega.rs:2842-2868), output * out_scale. qkv = q[32][128] | k[4][128] | v[4][128]. */
void oref_dattn_attend(oref_dattn *c, int layer, int pos, const float *qkv, float eps,
                       float out_scale, float *out);
void oref_dattn_read_row(const oref_dattn *c, int layer, int kv_head, int pos, uint16_t *k,
                         uint16_t *v);
void oref_dattn_write_rows(oref_dattn *c, int layer, int kv_head, int pos, int count,
                           const uint16_t *k, const uint16_t *v);

/* ---------------- whole decode step (Qwen3MoeOmegaEngine::step + logits) ---------------- */
typedef struct {
    int layers, hidden, q_heads, kv_heads, head_dim, experts, top_k, inter, vocab;
    float eps;
    double rope_theta;
} oref_config;

typedef struct oref_model oref_model;
/* Synthetic random-init model. sigma: projection weights; norm_sigma: norm weights are
 * 1 + N(0, norm_sigma) (0 gives exactly 1). Every tensor is generated eagerly (threads > 1
 * splits the work; the values do not depend on the thread count). */
oref_model *oref_model_synth(const oref_config *cfg, uint64_t seed, float sigma, float norm_sigma,
                             int threads);
/* The same model's layers layer_ids[0..cfg->layers) only: layer i of the result holds exactly the
 * tensors of layer layer_ids[i] of the model oref_model_synth makes with the same seed (the
 * embedding, lm_head and final norm as oref_model_synth makes them at cfg->vocab). Lets a check of
 * a few layers of a large model hold only those layers. */
oref_model *oref_model_synth_layers(const oref_config *cfg, uint64_t seed, float sigma,
                                    float norm_sigma, int threads, const int *layer_ids);
void oref_model_free(oref_model *m);
/* Raw views for upload. kind: 0 qkv, 1 o, 2 gate_up, 3 down (w and s), 4 router (bf16 in w),
 * 5 input_norm, 6 post_norm, 7 q_norm, 8 k_norm (f32 in w). Returns the pointer. */
const void *oref_model_tensor(const oref_model *m, int layer, int kind, const void **scale_out);
const uint16_t *oref_model_embed(const oref_model *m);
const uint16_t *oref_model_lm_head(const oref_model *m);
const float *oref_model_final_norm(const oref_model *m);

typedef struct oref_engine oref_engine;
oref_engine *oref_engine_new(const oref_model *m, int max_pos, int refined_router, int threads);
void oref_engine_free(oref_engine *e);
/* One token through every layer (qwen3_moe_omega.rs:4096-4345, fused attention and device
 * router arms). Writes the final-normed hidden (hidden floats); returns 0 or <0. */
int oref_engine_step(oref_engine *e, uint32_t token, float *hidden_out);
/* lm_head logits of a hidden row (qwen3_moe_omega.rs:4348-4368). */
void oref_engine_logits(oref_engine *e, const float *hidden, float *logits);
int oref_engine_pos(const oref_engine *e);
/* Benchmark support (no reference counterpart): position the engine at pos over the cache rows
 * 0..pos-1 as written through oref_engine_kv; returns 0 or -1 past the cache. */
int oref_engine_seek(oref_engine *e, int pos);
oref_dattn *oref_engine_kv(oref_engine *e);
/* Per-layer trace of the last step: routed ids/weights and the rank-8 / rank-9 logit margin. */
void oref_engine_last_routes(const oref_engine *e, uint32_t *ids, float *weights, float *margins);
/* Residual row after the last step (hidden floats). */
void oref_engine_last_x(const oref_engine *e, float *x);
/* Planted wiring mistakes (test infrastructure; 0 = none): 1 input / post-attention norm
 * weights swapped in oref_engine_step, 2 q rotated at pos + 1 in oref_dattn_attend (k at pos),
 * 3 the K/V row appended one slot late. Process-wide. */
void oref_set_mutant(int m);

#ifdef __cplusplus
}
#endif
#endif
