/* A C consumer of the static archive: built by gcc against include/omega_gpu.h and linked as
 * the reference's crates link the engine archive (their build.rs: -lomega_gpu plus the HIP
 * runtime, the C++ runtime, pthread and libm). On a host without a GPU each hot entry, given
 * valid arguments, must answer CHIP_FAIL with a message in its family's last_error; the checks
 * that run before any device call must answer as they do with a GPU. Prints one line per check;
 * the exit status is the number of failed checks. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "omega_gpu.h"

static int failures;

static void check(const char *what, int rc, int want, const char *err) {
    int ok = rc == want && (want == OMEGA_GPU_OK ? 1 : err != NULL && err[0] != '\0');
    printf("%s %s rc=%d (%s) last_error=%s\n", ok ? "ok" : "FAIL", what, rc,
           omega_gpu_fp8_rc_name(rc), err ? err : "(null)");
    if (!ok) failures++;
}

/* the call runs before its family's last_error is read (C leaves argument order open) */
#define EXPECT(what, call, want, last_error_fn)                                                  \
    do {                                                                                         \
        int rc_ = (call);                                                                        \
        check(what, rc_, want, last_error_fn());                                                 \
    } while (0)

static const char *no_error(void) { return NULL; }

int main(void) {
    /* host-side rules: no device involved */
    EXPECT("fp8_prepare(4096)", omega_gpu_fp8_prepare(4096), OMEGA_GPU_OK, no_error);
    EXPECT("fp8_prepare(100)", omega_gpu_fp8_prepare(100), OMEGA_GPU_BAD_ARGS,
           omega_gpu_fp8_last_error);
    EXPECT("bf16_prepare(100)", omega_gpu_bf16_prepare(100), OMEGA_GPU_BAD_ARGS,
           omega_gpu_bf16_last_error);
    if (strcmp(omega_gpu_fp8_rc_name(OMEGA_GPU_CHIP_FAIL), "CHIP_FAIL") != 0) failures++;

    /* FP8 expert weights: one 128 x 128 projection, unit scales */
    uint8_t *w8 = calloc(128 * 128, 1);
    uint16_t s8 = 0x3f80; /* 1.0 in bf16 */
    OmegaGpuFp8Tensor *ft = NULL;
    EXPECT("fp8_tensor_upload", omega_gpu_fp8_tensor_upload(1, 128, 128, w8, &s8, &ft),
           OMEGA_GPU_CHIP_FAIL, omega_gpu_fp8_last_error);
    if (ft != NULL) failures++;

    /* bf16 lm_head rows (k a multiple of 256) */
    uint16_t *wb = calloc(128 * 256, 2);
    OmegaGpuBf16Tensor *bt = NULL;
    EXPECT("bf16_tensor_upload", omega_gpu_bf16_tensor_upload(128, 256, wb, &bt),
           OMEGA_GPU_CHIP_FAIL, omega_gpu_bf16_last_error);
    if (bt != NULL) failures++;

    /* router and decode-attention state */
    OmegaGpuRouter *r = NULL;
    EXPECT("router_alloc_shape", omega_gpu_router_alloc_shape(48, 128, 0, &r),
           OMEGA_GPU_CHIP_FAIL, omega_gpu_router_last_error);
    OmegaGpuDecodeAttnCache *dc = NULL;
    EXPECT("decode_attn_cache_alloc", omega_gpu_decode_attn_cache_alloc(48, 4096, 1e6, &dc),
           OMEGA_GPU_CHIP_FAIL, omega_gpu_decode_attn_last_error);

    /* paged attention over a host KV pool of two 16-token blocks, one layer, 4 kv heads */
    OmegaGpuKvLayout lay;
    memset(&lay, 0, sizeof lay);
    lay.head_stride_bytes = 128 * 2;
    lay.token_stride_bytes = 4 * lay.head_stride_bytes;
    lay.kv_plane_stride_bytes = 16 * lay.token_stride_bytes;
    lay.layer_stride_bytes = 2 * lay.kv_plane_stride_bytes;
    lay.block_stride_bytes = lay.layer_stride_bytes;
    lay.pool_bytes = 2 * lay.block_stride_bytes;
    lay.num_blocks = 2;
    lay.num_layers = 1;
    lay.block_size = 16;
    void *pool = calloc(1, (size_t)lay.pool_bytes);
    float *q = calloc(32 * 128, sizeof(float));
    float *out = calloc(32 * 128, sizeof(float));
    uint32_t blocks[2] = {0, 1};
    EXPECT("paged_attention_bf16",
           omega_gpu_paged_attention_bf16(q, pool, &lay, blocks, 2, 20, 0, 32, 4, 128, out, NULL),
           OMEGA_GPU_CHIP_FAIL, omega_gpu_attention_last_error);
    int32_t tables[2] = {0, 1}, lens[1] = {20};
    EXPECT("paged_attention_batch_bf16",
           omega_gpu_paged_attention_batch_bf16(q, pool, &lay, tables, lens, 2, 1, 0, 32, 4, 128,
                                                out, NULL),
           OMEGA_GPU_CHIP_FAIL, omega_gpu_attention_last_error);

    /* the serving reservation opens the device */
    OmegaGpuServingBounds sb;
    memset(&sb, 0, sizeof sb);
    sb.max_context = 640;
    sb.max_seqs = 4;
    sb.num_q_heads = 32;
    sb.num_kv_heads = 4;
    sb.head_dim = 128;
    sb.kv_block_size = 16;
    sb.max_rows = 1;
    sb.max_k = 2048;
    sb.max_n = 2048;
    sb.kernel_slots = 8;
    EXPECT("reserve_serving", omega_gpu_reserve_serving(&sb), OMEGA_GPU_CHIP_FAIL,
           omega_gpu_matmul_last_error);

    /* a decode graph needs device handles: refused before any device call */
    OmegaGpuDecodeGraphConfig cfg;
    memset(&cfg, 0, sizeof cfg);
    cfg.layers = 48;
    cfg.vocab = 151936;
    cfg.eps = 1e-6f;
    OmegaGpuDecodeGraph *g = NULL;
    EXPECT("decode_graph_create(no handles)", omega_gpu_decode_graph_create(&cfg, &g),
           OMEGA_GPU_BAD_ARGS, omega_gpu_session_last_error);

    free(w8);
    free(wb);
    free(pool);
    free(q);
    free(out);
    printf("%d failed\n", failures);
    return failures;
}
