/*
 * CPU ORACLE — TEST INFRASTRUCTURE ONLY (see oracle.h). Never linked by the product library.
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp).
 * Reference paths are relative to the aien-dev/aien-sovereign-core-mv repository root;
 * "inference-abi/" abbreviates crates/aien-inference-abi/src/.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ======================================================================= codecs */

/* inference-abi/qwen3_moe.rs:481-483 */
float oref_bf16_to_f32(uint16_t bits) { return u2f((uint32_t)bits << 16); }

/* inference-abi/qwen3_moe.rs:486-493: RNE; NaN keeps NaN (quiet bit forced) */
uint16_t oref_f32_to_bf16(float v) {
    uint32_t bits = f2u(v);
    if (isnan(v)) return (uint16_t)((bits >> 16) | 0x40);
    uint32_t rounding = 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)((bits + rounding) >> 16);
}

/* crates/aien-kv-cache/src/lib.rs:116-121: RNE with a wrapping add, no NaN arm */
uint16_t oref_kv_f32_to_bf16(float v) {
    uint32_t u = f2u(v);
    uint32_t lsb = (u >> 16) & 1u;
    return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

/* inference-abi/qwen3_moe.rs:496-508: bias 7, no infinities, 0x7f / 0xff are NaN */
float oref_e4m3_to_f32(uint8_t bits) {
    float sign = (bits & 0x80) ? -1.0f : 1.0f;
    int exponent = (bits >> 3) & 0x0f;
    float mantissa = (float)(bits & 0x07);
    if (exponent == 0x0f && (bits & 0x07) == 0x07) return NAN;
    if (exponent == 0) return sign * mantissa * ldexpf(1.0f, -9);
    return sign * (1.0f + mantissa / 8.0f) * ldexpf(1.0f, exponent - 7);
}

/* inference-abi/qwen3_moe.rs:515-547: RNE, saturating at +-448, NaN -> 0x7f. The positive codes
 * 0x00..=0x7e increase with value; a binary search finds the bracketing pair, ties go to the even
 * code. */
uint8_t oref_f32_to_e4m3(float value) {
    if (isnan(value)) return 0x7f;
    uint8_t sign = signbit(value) ? 0x80 : 0;
    float magnitude = fabsf(value);
    uint8_t lo = 0, hi = 0x7e;
    if (magnitude >= oref_e4m3_to_f32(hi)) return sign | hi;
    while (hi - lo > 1) {
        uint8_t mid = lo + (hi - lo) / 2;
        if (oref_e4m3_to_f32(mid) <= magnitude) lo = mid; else hi = mid;
    }
    float below = oref_e4m3_to_f32(lo), above = oref_e4m3_to_f32(hi);
    float dl = magnitude - below, dh = above - magnitude;
    uint8_t code;
    if (dl < dh) code = lo;
    else if (dl > dh) code = hi;
    else code = (lo & 1) == 0 ? lo : hi;
    return sign | code;
}

/* The same rounding as oref_f32_to_e4m3 by bit arithmetic (the generator and the device-side
 * generator use this form; tests check it against the binary search). */
uint8_t oref_f32_to_e4m3_fast(float value) {
    if (isnan(value)) return 0x7f;
    uint32_t u = f2u(value);
    uint8_t sign = (u >> 31) ? 0x80 : 0;
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x43e00000u) return sign | 0x7e;            /* >= 448 */
    if (a < 0x3c800000u) {                                /* < 2^-6: multiples of 2^-9 */
        float m = u2f(a) * 512.0f;                        /* exact */
        return sign | (uint8_t)rintf(m);                  /* ties to even */
    }
    uint32_t e = (a >> 23) - 127 + 7;                     /* 1..15 */
    uint32_t mant = a & 0x7fffffu;
    uint32_t r = mant + 0x7ffffu + ((mant >> 20) & 1u);  /* RNE to 3 bits */
    uint32_t code = (e << 3) + (r >> 20);
    if (code > 0x7e) code = 0x7e;
    return sign | (uint8_t)code;
}

/* inference-abi/qwen3_moe_omega_prefill/fake_quant.rs:29-57 */
uint8_t oref_e4m3_rne_sat(float f) {
    uint8_t s = signbit(f) ? 0x80 : 0;
    double a = fabs((double)f);
    if (isinf(f) || a > 448.0) return s | 0x7e;
    if (a < ldexp(1.0, -6)) return s | (uint8_t)nearbyint(a * 512.0);
    int e = (int)floor(log2(a));
    double m = a / ldexp(1.0, e);
    if (m >= 2.0) { e += 1; m /= 2.0; }
    else if (m < 1.0) { e -= 1; m *= 2.0; }
    int mm = (int)nearbyint((m - 1.0) * 8.0);
    if (mm >= 8) { mm = 0; e += 1; }
    if (e + 7 > 15 || (((e + 7) << 3) | mm) > 0x7e) return s | 0x7e;
    return s | (uint8_t)(((e + 7) << 3) | mm);
}

/* fake_quant.rs:60-72 */
float oref_fq_e4m3_to_f32(uint8_t c) {
    int s = c >> 7, e = (c >> 3) & 15;
    float mm = (float)(c & 7);
    float v = e != 0 ? (1.0f + mm / 8.0f) * ldexpf(1.0f, e - 7) : (mm / 8.0f) * ldexpf(1.0f, -6);
    return s ? -v : v;
}

/* fake_quant.rs:75-83: a power-of-two scale from the block amax (the exponent rounds up when the
 * mantissa is above 1.75) */
void oref_block_scale(float m, float *scale, float *inv) {
    uint32_t mb = f2u(m);
    uint32_t e = mb >> 23, mant = mb & 0x7fffffu;
    uint32_t c = (mant + 0x1fffffu) >> 23;
    *scale = u2f((e + c - 8) << 23);
    *inv = u2f((262 - e - c) << 23);
}

/* fake_quant.rs:87-106 */
void oref_quant_row(const float *x, int k, uint8_t *q, float *s) {
    for (int b = 0; b < k / 128; b++) {
        const float *blk = x + b * 128;
        float m = ldexpf(1.0f, -100);
        for (int j = 0; j < 128; j++) m = fmaxf(m, fabsf(blk[j]));
        float scale, inv;
        oref_block_scale(m, &scale, &inv);
        s[b] = scale;
        for (int j = 0; j < 128; j++) q[b * 128 + j] = oref_e4m3_rne_sat(blk[j] * inv);
    }
}

/* fake_quant.rs:109-117 */
void oref_fake_quant_row(float *x, int k) {
    uint8_t *q = malloc((size_t)k);
    float *s = malloc(sizeof(float) * (size_t)(k / 128));
    oref_quant_row(x, k, q, s);
    for (int j = 0; j < k; j++) x[j] = oref_fq_e4m3_to_f32(q[j]) * s[j / 128];
    free(q);
    free(s);
}

/* fake_quant.rs:120-124 */
void oref_bf16_round_row(float *x, int k) {
    for (int j = 0; j < k; j++) x[j] = oref_bf16_to_f32(oref_f32_to_bf16(x[j]));
}

/* inference-abi/qwen3_moe.rs:559-567 (OracleActivations::Fp8Block128) */
void oref_quantize_block128(float *x, int k) {
    for (int b = 0; b < k; b += 128) {
        int n = k - b < 128 ? k - b : 128;
        float maximum = 0.0f;
        for (int j = 0; j < n; j++) maximum = fmaxf(maximum, fabsf(x[b + j]));
        float scale = maximum > 0.0f ? maximum / 448.0f : 1.0f;
        for (int j = 0; j < n; j++)
            x[b + j] = oref_e4m3_to_f32(oref_f32_to_e4m3(x[b + j] / scale)) * scale;
    }
}

/* =================================================================== generators */

/* inference-abi/qwen3_moe_omega.rs:1654-1662 */
float oref_prand(uint64_t seed, uint64_t idx) {
    uint64_t x = seed * 0x9E3779B97F4A7C15ull + (idx + 1);
    x ^= x >> 29;
    x *= 0xBF58476D1CE4E5B9ull;
    x ^= x >> 32;
    return ((float)(x & 0xFFFF) / 32768.0f) - 1.0f;
}

uint64_t oref_splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

float oref_synth_normal(uint64_t seed, uint64_t tensor, uint64_t idx, float sigma) {
    uint64_t base = oref_splitmix64(seed ^ (tensor * 0xD1B54A32D192ED03ull)) + idx * 3;
    int32_t sum = 0;
    for (int j = 0; j < 3; j++) {
        uint64_t h = oref_splitmix64(base + (uint64_t)j);
        sum += (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) +
               (int32_t)((h >> 32) & 0xffff) + (int32_t)((h >> 48) & 0xffff);
    }
    float c = sigma * (1.0f / 65536.0f);
    return (float)(sum - 393210) * c;
}

void oref_synth_bf16(uint64_t seed, uint64_t tensor, size_t count, float sigma, int one_plus,
                     uint16_t *out) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < count; i++) {
        float v = oref_synth_normal(seed, tensor, i, sigma);
        if (one_plus) v = 1.0f + v;
        out[i] = oref_f32_to_bf16(v);
    }
}

void oref_synth_f32(uint64_t seed, uint64_t tensor, size_t count, float sigma, int one_plus,
                    float *out) {
    for (size_t i = 0; i < count; i++) {
        float v = oref_synth_normal(seed, tensor, i, sigma);
        out[i] = one_plus ? 1.0f + v : v;
    }
}

void oref_synth_fp8(uint64_t seed, uint64_t tensor, int experts, int n, int k, float sigma,
                    uint8_t *w, uint16_t *scale_bf16) {
    int nb = n / 128, kb = k / 128;
#pragma omp parallel for collapse(3) schedule(static)
    for (int e = 0; e < experts; e++)
        for (int rb = 0; rb < nb; rb++)
            for (int cb = 0; cb < kb; cb++) {
                float amax = 0.0f;
                size_t ebase = (size_t)e * n * k;
                for (int r = 0; r < 128; r++)
                    for (int c = 0; c < 128; c++) {
                        size_t idx = ebase + (size_t)(rb * 128 + r) * k + cb * 128 + c;
                        amax = fmaxf(amax, fabsf(oref_synth_normal(seed, tensor, idx, sigma)));
                    }
                uint16_t sb = oref_f32_to_bf16(amax / 448.0f);
                float s = oref_bf16_to_f32(sb);
                scale_bf16[((size_t)e * nb + rb) * kb + cb] = sb;
                for (int r = 0; r < 128; r++)
                    for (int c = 0; c < 128; c++) {
                        size_t idx = ebase + (size_t)(rb * 128 + r) * k + cb * 128 + c;
                        float v = oref_synth_normal(seed, tensor, idx, sigma);
                        w[idx] = oref_f32_to_e4m3_fast(v / s);
                    }
            }
}

/* ==================================================================== FP8 GEMV */

static float g_lut[256];
static int g_lut_ready = 0;
static const float *lut(void) {
    if (!g_lut_ready) {
        for (int b = 0; b < 256; b++) g_lut[b] = oref_e4m3_to_f32((uint8_t)b);
        g_lut_ready = 1;
    }
    return g_lut;
}

/* one row of HostFp8::grouped_f32 (inference-abi/qwen3_moe_omega.rs:2129-2136) */
static float fp8_row(const uint8_t *wr, const uint16_t *srow, int k, const float *x,
                     const float *L) {
    float acc = 0.0f;
    for (int c = 0; c < k; c++) {
        float t = L[wr[c]] * oref_bf16_to_f32(srow[c / 128]);
        acc += t * x[c];
    }
    return acc;
}

static void fp8_grouped_impl(const uint8_t *w, const uint16_t *s, int experts, int n, int k,
                             int groups, const uint32_t *ids, const float *x, int x_rows,
                             float *y, int threads) {
    const float *L = lut();
    int kb = k / 128;
    (void)experts;
#pragma omp parallel for collapse(2) schedule(static) num_threads(threads > 0 ? threads : 1)
    for (int g = 0; g < groups; g++)
        for (int r = 0; r < n; r++) {
            size_t id = ids[g];
            const float *xr = x_rows == 1 ? x : x + (size_t)g * k;
            const uint8_t *we = w + id * (size_t)n * k;
            const uint16_t *se = s + id * (size_t)(n / 128) * kb;
            y[(size_t)g * n + r] = fp8_row(we + (size_t)r * k, se + (size_t)(r / 128) * kb, k, xr, L);
        }
}

/* inference-abi/qwen3_moe_omega.rs:2114-2139 */
void oref_fp8_grouped(const uint8_t *w, const uint16_t *s, int experts, int n, int k, int groups,
                      const uint32_t *ids, const float *x, int x_rows, float *y) {
    fp8_grouped_impl(w, s, experts, n, k, groups, ids, x, x_rows, y, 1);
}

void oref_fp8_grouped_mt(const uint8_t *w, const uint16_t *s, int experts, int n, int k,
                         int groups, const uint32_t *ids, const float *x, int x_rows, float *y,
                         int threads) {
    fp8_grouped_impl(w, s, experts, n, k, groups, ids, x, x_rows, y, threads);
}

/* inference-abi/qwen3_moe.rs:595-619 */
void oref_dequant_matvec(const uint8_t *w, const uint16_t *s, int rows, int cols, const float *v,
                         float *out) {
    const float *L = lut();
    int kb = cols / 128;
    for (int r = 0; r < rows; r++) {
        const uint8_t *row = w + (size_t)r * cols;
        float total = 0.0f;
        for (int b = 0; b < kb; b++) {
            float dot = 0.0f;
            for (int j = 0; j < 128; j++) dot += L[row[b * 128 + j]] * v[b * 128 + j];
            total += dot * oref_bf16_to_f32(s[(r / 128) * kb + b]);
        }
        out[r] = total;
    }
}

static void bf16_gemv_impl(const uint16_t *w, int n, int k, const float *x, float *y, int threads) {
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
    for (int r = 0; r < n; r++) {
        const uint16_t *wr = w + (size_t)r * k;
        float acc = 0.0f;
        for (int c = 0; c < k; c++) acc += oref_bf16_to_f32(wr[c]) * x[c];
        y[r] = acc;
    }
}

/* inference-abi/qwen3_moe_omega.rs:2015-2028 */
void oref_bf16_gemv(const uint16_t *w, int n, int k, const float *x, float *y) {
    bf16_gemv_impl(w, n, k, x, y, 1);
}
void oref_bf16_gemv_mt(const uint16_t *w, int n, int k, const float *x, float *y, int threads) {
    bf16_gemv_impl(w, n, k, x, y, threads);
}

/* inference-abi/tensor.rs:299-318 (the index; the logprob is not on the path) */
uint32_t oref_argmax(const float *logits, int n) {
    int best = 0;
    float bv = logits[0];
    for (int i = 1; i < n; i++)
        if (logits[i] > bv) { bv = logits[i]; best = i; }
    return (uint32_t)best;
}

/* ============================================================ norms, rope, attention */

/* inference-abi/tensor.rs:94-110: f64 sum of squares, f32 scale, out = x * scale * w */
void oref_rmsnorm(const float *x, const float *w, int dim, float eps, float *out) {
    double sum_sq = 0.0;
    for (int i = 0; i < dim; i++) {
        double vf = (double)x[i];
        sum_sq += vf * vf;
    }
    double mean_sq = sum_sq / (double)dim;
    float scale = (float)(1.0 / sqrt(mean_sq + (double)eps));
    for (int i = 0; i < dim; i++) out[i] = x[i] * scale * w[i];
}

/* inference-abi/qwen3_coder.rs:306-320 */
void oref_rmsnorm_per_head(const float *x, const float *w, float eps, int heads, int hd,
                           float *out) {
    for (int h = 0; h < heads; h++) oref_rmsnorm(x + h * hd, w, hd, eps, out + h * hd);
}

/* inference-abi/tensor.rs:150-161; inv_freq from crates/aien-abi-core/src/lib.rs:106-113 */
void oref_rope_cos_sin(double theta, int hd, int pos, float *cos_out, float *sin_out) {
    int half = hd / 2;
    for (int i = 0; i < half; i++) {
        double exponent = (double)(2 * i) / (double)hd;
        double inv_freq = 1.0 / pow(theta, exponent);
        double rot = (double)pos * inv_freq;
        sin_out[i] = (float)sin(rot);
        cos_out[i] = (float)cos(rot);
    }
}

/* inference-abi/tensor.rs:164-190: rotate_half pairs (i, i + hd/2) */
void oref_apply_rope(float *q, float *k, int pos, int qh, int kvh, int hd, double theta) {
    int half = hd / 2;
    float *cs = malloc(sizeof(float) * (size_t)hd);
    float *sn = cs + half;
    oref_rope_cos_sin(theta, hd, pos, cs, sn);
    float *vs[2] = {q, k};
    int heads[2] = {qh, kvh};
    for (int t = 0; t < 2; t++)
        for (int h = 0; h < heads[t]; h++) {
            float *v = vs[t] + h * hd;
            for (int i = 0; i < half; i++) {
                float v0 = v[i], v1 = v[i + half];
                v[i] = v0 * cs[i] - v1 * sn[i];
                v[i + half] = v0 * sn[i] + v1 * cs[i];
            }
        }
    free(cs);
}

/* inference-abi/tensor.rs:193-250 */
void oref_sdpa(const float *q, const float *k, const float *v, int ctx, int qh, int kvh, int hd,
               float *out) {
    if (ctx == 0) {
        memset(out, 0, sizeof(float) * (size_t)qh * hd);
        return;
    }
    int ratio = qh / kvh;
    int kvd = kvh * hd;
    double inv_sqrt_d = 1.0 / sqrt((double)hd);
    double *scores = malloc(sizeof(double) * (size_t)ctx);
    for (int h = 0; h < qh; h++) {
        int kv = h / ratio;
        const float *qhd = q + h * hd;
        for (int t = 0; t < ctx; t++) {
            const float *kt = k + (size_t)t * kvd + kv * hd;
            double dot = 0.0;
            for (int d = 0; d < hd; d++) dot += (double)qhd[d] * (double)kt[d];
            scores[t] = dot * inv_sqrt_d;
        }
        double mx = -INFINITY;
        for (int t = 0; t < ctx; t++) mx = fmax(mx, scores[t]);
        double sum_exp = 0.0;
        for (int t = 0; t < ctx; t++) {
            scores[t] = exp(scores[t] - mx);
            sum_exp += scores[t];
        }
        double inv_sum = 1.0 / fmax(sum_exp, 1e-12);
        for (int t = 0; t < ctx; t++) scores[t] *= inv_sum;
        for (int d = 0; d < hd; d++) {
            double sum = 0.0;
            for (int t = 0; t < ctx; t++) sum += scores[t] * (double)v[(size_t)t * kvd + kv * hd + d];
            out[h * hd + d] = (float)sum;
        }
    }
    free(scores);
}

/* ============================================================== routing and MoE */

/* qwen3_moe_omega.rs:1968-1976 (FakeRouter) and :5637-5650 (router_logits) */
void oref_router_logits(const uint16_t *gate_bf16, const float *post, int experts, int hidden,
                        float *logits) {
    for (int e = 0; e < experts; e++) {
        const uint16_t *g = gate_bf16 + (size_t)e * hidden;
        float acc = 0.0f;
        for (int c = 0; c < hidden; c++) acc += oref_bf16_to_f32(g[c]) * post[c];
        logits[e] = acc;
    }
}

/* Refinement, not in the reference: exact f32 products accumulated in f64, one rounding. */
void oref_router_logits_f64(const uint16_t *gate_bf16, const float *post, int experts, int hidden,
                            float *logits) {
    for (int e = 0; e < experts; e++) {
        const uint16_t *g = gate_bf16 + (size_t)e * hidden;
        double acc = 0.0;
        for (int c = 0; c < hidden; c++) acc += (double)oref_bf16_to_f32(g[c]) * (double)post[c];
        logits[e] = (float)acc;
    }
}

/* f32::total_cmp as a signed key (NaN never reaches it: from_logits refuses non-finite) */
static inline int32_t total_key(float f) {
    int32_t b = (int32_t)f2u(f);
    return b < 0 ? (int32_t)((uint32_t)b ^ 0x7fffffffu) : b;
}

/* moe_plan.rs:86-171 */
int oref_moe_plan(const float *logits, int tokens, int experts, int top_k, uint32_t *topk_experts,
                  float *topk_weights, uint32_t *expert_offsets, uint32_t *grouped_to_assignment,
                  uint32_t *assignment_to_grouped, uint32_t *grouped_token_ids) {
    if (experts <= 0 || top_k <= 0 || top_k > experts || tokens < 0) return -1;
    int assignments = tokens * top_k;
    uint32_t *counts = calloc((size_t)experts, sizeof(uint32_t));
    int *ranking = malloc(sizeof(int) * (size_t)experts);
    float *sel = malloc(sizeof(float) * (size_t)top_k);
    for (int t = 0; t < tokens; t++) {
        const float *row = logits + (size_t)t * experts;
        for (int e = 0; e < experts; e++)
            if (!isfinite(row[e])) {
                free(counts); free(ranking); free(sel);
                return -(2 + t * experts + e);
            }
        /* descending by total_cmp, ties to the lower id: an insertion sort of the ids keeps the
         * comparator's total order exactly (the comparator itself is a total order, so the sorted
         * sequence is unique whatever algorithm produces it) */
        for (int e = 0; e < experts; e++) {
            int j = e;
            int32_t ke = total_key(row[e]);
            while (j > 0) {
                int p = ranking[j - 1];
                int32_t kp = total_key(row[p]);
                if (kp > ke || (kp == ke && p < e)) break;
                ranking[j] = p;
                j--;
            }
            ranking[j] = e;
        }
        float max_logit = row[ranking[0]];
        float sum = 0.0f;
        for (int s = 0; s < top_k; s++) {
            float p = expf(row[ranking[s]] - max_logit);
            sel[s] = p;
            sum += p;
        }
        for (int s = 0; s < top_k; s++) {
            int e = ranking[s];
            topk_experts[t * top_k + s] = (uint32_t)e;
            topk_weights[t * top_k + s] = sel[s] / sum;
            counts[e]++;
        }
    }
    if (expert_offsets) {
        expert_offsets[0] = 0;
        for (int e = 0; e < experts; e++) expert_offsets[e + 1] = expert_offsets[e] + counts[e];
        uint32_t *cursor = malloc(sizeof(uint32_t) * (size_t)experts);
        memcpy(cursor, expert_offsets, sizeof(uint32_t) * (size_t)experts);
        for (int a = 0; a < assignments; a++) {
            uint32_t e = topk_experts[a];
            uint32_t g = cursor[e]++;
            if (grouped_to_assignment) grouped_to_assignment[g] = (uint32_t)a;
            if (assignment_to_grouped) assignment_to_grouped[a] = g;
            if (grouped_token_ids) grouped_token_ids[g] = (uint32_t)(a / top_k);
        }
        free(cursor);
    }
    free(counts);
    free(ranking);
    free(sel);
    return 0;
}

/* moe_plan.rs:213-233 */
void oref_reduce_grouped(const uint32_t *assignment_to_grouped, const float *topk_weights,
                         int tokens, int top_k, const float *grouped, int hidden, float *out) {
    memset(out, 0, sizeof(float) * (size_t)tokens * hidden);
    for (int a = 0; a < tokens * top_k; a++) {
        size_t g = assignment_to_grouped[a];
        int t = a / top_k;
        float w = topk_weights[a];
        for (int c = 0; c < hidden; c++) out[(size_t)t * hidden + c] += grouped[g * hidden + c] * w;
    }
}

/* qwen3_moe_omega.rs:5616-5621 */
void oref_swiglu(const float *gu, int i, float *act) {
    for (int j = 0; j < i; j++) {
        float g = gu[j];
        act[j] = g / (1.0f + expf(-g)) * gu[i + j];
    }
}

/* qwen3_moe_omega.rs:1943-1998 */
int oref_route(const uint16_t *gate_bf16, const float *norm_w, int experts, int hidden, int top_k,
               const float *x, float eps, int refined, uint32_t *ids, float *weights, float *post,
               float *logits) {
    float *p = post ? post : malloc(sizeof(float) * (size_t)hidden);
    float *l = logits ? logits : malloc(sizeof(float) * (size_t)experts);
    oref_rmsnorm(x, norm_w, hidden, eps, p);
    if (refined) oref_router_logits_f64(gate_bf16, p, experts, hidden, l);
    else oref_router_logits(gate_bf16, p, experts, hidden, l);
    int rc = oref_moe_plan(l, 1, experts, top_k, ids, weights, NULL, NULL, NULL, NULL);
    if (!post) free(p);
    if (!logits) free(l);
    return rc;
}

/* qwen3_moe.rs:626-686 */
void oref_moe_forward(const uint8_t *gu_w, const uint16_t *gu_s, const uint8_t *dn_w,
                      const uint16_t *dn_s, int h, int i, int tokens, int top_k,
                      const uint32_t *topk_experts, const float *topk_weights, const float *x,
                      int quantize, float *out) {
    size_t gu_scale_len = (size_t)(2 * i / 128) * (h / 128);
    size_t dn_scale_len = (size_t)(h / 128) * (i / 128);
    memset(out, 0, sizeof(float) * (size_t)tokens * h);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < tokens; t++) {
        float *xt = malloc(sizeof(float) * (size_t)h);
        float *proj = malloc(sizeof(float) * (size_t)2 * i);
        float *hid = malloc(sizeof(float) * (size_t)i);
        float *eo = malloc(sizeof(float) * (size_t)h);
        memcpy(xt, x + (size_t)t * h, sizeof(float) * (size_t)h);
        if (quantize) oref_quantize_block128(xt, h);
        for (int slot = 0; slot < top_k; slot++) {
            size_t e = topk_experts[t * top_k + slot];
            float weight = topk_weights[t * top_k + slot];
            oref_dequant_matvec(gu_w + e * 2 * (size_t)i * h, gu_s + e * gu_scale_len, 2 * i, h,
                                xt, proj);
            for (int j = 0; j < i; j++) {
                float g = proj[j];
                hid[j] = g / (1.0f + expf(-g)) * proj[i + j];
            }
            if (quantize) oref_quantize_block128(hid, i);
            oref_dequant_matvec(dn_w + e * (size_t)h * i, dn_s + e * dn_scale_len, h, i, hid, eo);
            for (int c = 0; c < h; c++) out[(size_t)t * h + c] += weight * eo[c];
        }
        free(xt); free(proj); free(hid); free(eo);
    }
}

/* qwen3_moe_omega.rs:4287-4318 (FP8 grouped arm) with the W8A8 control's rounding
 * (qwen3_moe_omega/w8a8_control.rs:21-25, 161-171) */
void oref_moe_block(const uint8_t *gu_w, const uint16_t *gu_s, const uint8_t *dn_w,
                    const uint16_t *dn_s, int experts, int h, int i, int top_k,
                    const uint32_t *ids, const float *weights, const float *post, int w8a8,
                    float *moe_out) {
    float *xin = malloc(sizeof(float) * (size_t)h);
    float *gu = malloc(sizeof(float) * (size_t)top_k * 2 * i);
    float *act = malloc(sizeof(float) * (size_t)top_k * i);
    float *dn = malloc(sizeof(float) * (size_t)top_k * h);
    memcpy(xin, post, sizeof(float) * (size_t)h);
    if (w8a8) oref_fake_quant_row(xin, h);
    fp8_grouped_impl(gu_w, gu_s, experts, 2 * i, h, top_k, ids, xin, 1, gu, 1);
    for (int s = 0; s < top_k; s++) {
        oref_swiglu(gu + (size_t)s * 2 * i, i, act + (size_t)s * i);
        if (w8a8) {
            oref_bf16_round_row(act + (size_t)s * i, i);
            oref_fake_quant_row(act + (size_t)s * i, i);
        }
    }
    fp8_grouped_impl(dn_w, dn_s, experts, h, i, top_k, ids, act, top_k, dn, 1);
    for (int c = 0; c < h; c++) moe_out[c] = 0.0f;
    for (int s = 0; s < top_k; s++)
        for (int c = 0; c < h; c++) moe_out[c] += weights[s] * dn[(size_t)s * h + c];
    free(xin); free(gu); free(act); free(dn);
}

/* ============================================================== KV page layout */

/* crates/aien-kv-cache/src/lib.rs:247-292 (bf16 elements) */
void oref_kv_layout_bf16(uint32_t num_blocks, uint32_t block_size, uint32_t layers,
                         uint32_t kv_heads, uint32_t head_dim, oref_kv_layout *o) {
    o->head_stride_bytes = (uint64_t)head_dim * 2;
    o->token_stride_bytes = (uint64_t)kv_heads * o->head_stride_bytes;
    o->kv_plane_stride_bytes = (uint64_t)block_size * o->token_stride_bytes;
    o->layer_stride_bytes = 2 * o->kv_plane_stride_bytes;
    o->block_stride_bytes = (uint64_t)layers * o->layer_stride_bytes;
    o->pool_bytes = (uint64_t)num_blocks * o->block_stride_bytes;
    o->num_blocks = num_blocks;
    o->num_layers = layers;
    o->block_size = block_size;
}

/* lib.rs:294-316 */
uint64_t oref_kv_element_offset(const oref_kv_layout *l, uint32_t block, uint32_t layer,
                                int is_value, uint32_t token, uint32_t head, uint32_t dim) {
    return (uint64_t)block * l->block_stride_bytes + (uint64_t)layer * l->layer_stride_bytes +
           (is_value ? l->kv_plane_stride_bytes : 0) + (uint64_t)token * l->token_stride_bytes +
           (uint64_t)head * l->head_stride_bytes + (uint64_t)dim * 2;
}

/* lib.rs:586-622 */
void oref_kv_write_token(uint8_t *pool, const oref_kv_layout *l, uint32_t block, uint32_t layer,
                         uint32_t token, int kv_dim, const float *k, const float *v) {
    uint64_t ko = oref_kv_element_offset(l, block, layer, 0, token, 0, 0);
    uint64_t vo = oref_kv_element_offset(l, block, layer, 1, token, 0, 0);
    for (int i = 0; i < kv_dim; i++) {
        uint16_t kb = oref_kv_f32_to_bf16(k[i]), vb = oref_kv_f32_to_bf16(v[i]);
        memcpy(pool + ko + 2 * (uint64_t)i, &kb, 2);
        memcpy(pool + vo + 2 * (uint64_t)i, &vb, 2);
    }
}

/* lib.rs:624-659 */
void oref_kv_read_token(const uint8_t *pool, const oref_kv_layout *l, uint32_t block,
                        uint32_t layer, uint32_t token, int kv_dim, float *k, float *v) {
    uint64_t ko = oref_kv_element_offset(l, block, layer, 0, token, 0, 0);
    uint64_t vo = oref_kv_element_offset(l, block, layer, 1, token, 0, 0);
    for (int i = 0; i < kv_dim; i++) {
        uint16_t kb, vb;
        memcpy(&kb, pool + ko + 2 * (uint64_t)i, 2);
        memcpy(&vb, pool + vo + 2 * (uint64_t)i, 2);
        k[i] = oref_bf16_to_f32(kb);
        v[i] = oref_bf16_to_f32(vb);
    }
}

/* lib.rs:661-691 (gather) then tensor.rs:193-250 (attend), as HostPoolKv::attend does
 * (qwen3_moe_omega.rs:2842-2868) */
void oref_paged_attention(const float *q, const uint8_t *pool, const oref_kv_layout *l,
                          const int32_t *block_table, int context_len, int layer, int qh, int kvh,
                          int hd, float *out) {
    int kvd = kvh * hd;
    float *K = malloc(sizeof(float) * (size_t)(context_len > 0 ? context_len : 1) * kvd);
    float *V = malloc(sizeof(float) * (size_t)(context_len > 0 ? context_len : 1) * kvd);
    int read = 0;
    for (int b = 0; read < context_len; b++) {
        int in_block = context_len - read < (int)l->block_size ? context_len - read : (int)l->block_size;
        for (int t = 0; t < in_block; t++)
            oref_kv_read_token(pool, l, (uint32_t)block_table[b], (uint32_t)layer, (uint32_t)t, kvd,
                               K + (size_t)(read + t) * kvd, V + (size_t)(read + t) * kvd);
        read += in_block;
    }
    oref_sdpa(q, K, V, context_len, qh, kvh, hd, out);
    free(K);
    free(V);
}

/* qwen3_moe_omega.rs:5899-5903 (FNV-1a 64) */
uint64_t oref_fnv1a64(const uint8_t *bytes, size_t n) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < n; i++) h = (h ^ bytes[i]) * 0x00000100000001b3ull;
    return h;
}

/* ================================================================= fused decode attention */

#define DA_QH 32
#define DA_KVH 4
#define DA_HD 128

struct oref_dattn {
    int layers, max_pos;
    double theta;
    float *q_norm, *k_norm;   /* [layers][128] */
    uint16_t *k, *v;          /* [layers][kv_head][max_pos][128] */
};

oref_dattn *oref_dattn_alloc(int layers, int max_pos, double theta) {
    oref_dattn *c = calloc(1, sizeof(*c));
    c->layers = layers;
    c->max_pos = max_pos;
    c->theta = theta;
    c->q_norm = calloc((size_t)layers * DA_HD, sizeof(float));
    c->k_norm = calloc((size_t)layers * DA_HD, sizeof(float));
    size_t rows = (size_t)layers * DA_KVH * max_pos * DA_HD;
    c->k = calloc(rows, 2);
    c->v = calloc(rows, 2);
    return c;
}

void oref_dattn_free(oref_dattn *c) {
    if (!c) return;
    free(c->q_norm); free(c->k_norm); free(c->k); free(c->v);
    free(c);
}

void oref_dattn_set_norms(oref_dattn *c, int layer, const float *q_norm, const float *k_norm) {
    memcpy(c->q_norm + (size_t)layer * DA_HD, q_norm, sizeof(float) * DA_HD);
    memcpy(c->k_norm + (size_t)layer * DA_HD, k_norm, sizeof(float) * DA_HD);
}

static inline size_t da_row(const oref_dattn *c, int layer, int head, int pos) {
    return (((size_t)layer * DA_KVH + head) * c->max_pos + pos) * DA_HD;
}

/* Planted wiring mistakes for the composition checks (test infrastructure, off by default):
 * 1 the engine swaps the input and post-attention norm weights, 2 q is rotated at pos + 1 (k at
 * pos), 3 this token's K/V row is appended one slot late. */
static int g_mutant = 0;
void oref_set_mutant(int m) { g_mutant = m; }

void oref_dattn_attend(oref_dattn *c, int layer, int pos, const float *qkv, float eps,
                       float out_scale, float *out) {
    float q[DA_QH * DA_HD], k[DA_KVH * DA_HD];
    const float *v = qkv + DA_QH * DA_HD + DA_KVH * DA_HD;
    oref_rmsnorm_per_head(qkv, c->q_norm + (size_t)layer * DA_HD, eps, DA_QH, DA_HD, q);
    oref_rmsnorm_per_head(qkv + DA_QH * DA_HD, c->k_norm + (size_t)layer * DA_HD, eps, DA_KVH,
                          DA_HD, k);
    if (g_mutant == 2) {
        float kdummy[DA_KVH * DA_HD];
        memcpy(kdummy, k, sizeof(kdummy));
        oref_apply_rope(q, kdummy, pos + 1, DA_QH, DA_KVH, DA_HD, c->theta);
        float qdummy[DA_QH * DA_HD];
        memcpy(qdummy, q, sizeof(qdummy));
        oref_apply_rope(qdummy, k, pos, DA_QH, DA_KVH, DA_HD, c->theta);
    } else {
        oref_apply_rope(q, k, pos, DA_QH, DA_KVH, DA_HD, c->theta);
    }
    const int slot = g_mutant == 3 && pos + 1 < c->max_pos ? pos + 1 : pos;
    for (int h = 0; h < DA_KVH; h++)
        for (int d = 0; d < DA_HD; d++) {
            c->k[da_row(c, layer, h, slot) + d] = oref_kv_f32_to_bf16(k[h * DA_HD + d]);
            c->v[da_row(c, layer, h, slot) + d] = oref_kv_f32_to_bf16(v[h * DA_HD + d]);
        }
    int ctx = pos + 1;
    float *K = malloc(sizeof(float) * (size_t)ctx * DA_KVH * DA_HD);
    float *V = malloc(sizeof(float) * (size_t)ctx * DA_KVH * DA_HD);
    for (int t = 0; t < ctx; t++)
        for (int h = 0; h < DA_KVH; h++)
            for (int d = 0; d < DA_HD; d++) {
                K[((size_t)t * DA_KVH + h) * DA_HD + d] = oref_bf16_to_f32(c->k[da_row(c, layer, h, t) + d]);
                V[((size_t)t * DA_KVH + h) * DA_HD + d] = oref_bf16_to_f32(c->v[da_row(c, layer, h, t) + d]);
            }
    oref_sdpa(q, K, V, ctx, DA_QH, DA_KVH, DA_HD, out);
    if (out_scale != 1.0f)
        for (int i = 0; i < DA_QH * DA_HD; i++) out[i] *= out_scale;
    free(K);
    free(V);
}

void oref_dattn_read_row(const oref_dattn *c, int layer, int kv_head, int pos, uint16_t *k,
                         uint16_t *v) {
    memcpy(k, c->k + da_row(c, layer, kv_head, pos), 2 * DA_HD);
    memcpy(v, c->v + da_row(c, layer, kv_head, pos), 2 * DA_HD);
}

void oref_dattn_write_rows(oref_dattn *c, int layer, int kv_head, int pos, int count,
                           const uint16_t *k, const uint16_t *v) {
    memcpy(c->k + da_row(c, layer, kv_head, pos), k, 2 * (size_t)DA_HD * count);
    memcpy(c->v + da_row(c, layer, kv_head, pos), v, 2 * (size_t)DA_HD * count);
}

/* ================================================================= synthetic model */

struct oref_model {
    oref_config cfg;
    uint8_t **w[4];        /* qkv, o, gate_up, down (e4m3) */
    uint16_t **s[4];       /* their bf16 scales */
    uint16_t **router;     /* [experts][hidden] bf16 */
    float **norms[4];      /* input, post, q, k */
    uint16_t *embed, *lm_head;
    float *final_norm;
};

/* tensor ids of the generator: one per (layer, kind) plus the model-wide ones */
static uint64_t tid(int layer, int kind) { return 1000ull + (uint64_t)layer * 16 + (uint64_t)kind; }

oref_model *oref_model_synth_layers(const oref_config *c, uint64_t seed, float sigma,
                                    float norm_sigma, int threads, const int *layer_ids);

oref_model *oref_model_synth(const oref_config *c, uint64_t seed, float sigma, float norm_sigma,
                             int threads) {
    return oref_model_synth_layers(c, seed, sigma, norm_sigma, threads, NULL);
}

oref_model *oref_model_synth_layers(const oref_config *c, uint64_t seed, float sigma,
                                    float norm_sigma, int threads, const int *layer_ids) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
    oref_model *m = calloc(1, sizeof(*m));
    m->cfg = *c;
    int L = c->layers, h = c->hidden, hd = c->head_dim;
    int qkv_n = (c->q_heads + 2 * c->kv_heads) * hd, qd = c->q_heads * hd;
    int ns[4] = {qkv_n, h, 2 * c->inter, h}, ks[4] = {h, qd, h, c->inter};
    int es[4] = {1, 1, c->experts, c->experts};
    for (int t = 0; t < 4; t++) {
        m->w[t] = calloc((size_t)L, sizeof(void *));
        m->s[t] = calloc((size_t)L, sizeof(void *));
        m->norms[t] = calloc((size_t)L, sizeof(void *));
    }
    m->router = calloc((size_t)L, sizeof(void *));
    int norm_len[4] = {h, h, hd, hd};
    for (int l = 0; l < L; l++) {
        const int src = layer_ids ? layer_ids[l] : l;  /* the full model's layer this one holds */
        for (int t = 0; t < 4; t++) {
            size_t nw = (size_t)es[t] * ns[t] * ks[t];
            m->w[t][l] = malloc(nw);
            m->s[t][l] = malloc(sizeof(uint16_t) * (size_t)es[t] * (ns[t] / 128) * (ks[t] / 128));
            oref_synth_fp8(seed, tid(src, t), es[t], ns[t], ks[t], sigma, m->w[t][l], m->s[t][l]);
            m->norms[t][l] = malloc(sizeof(float) * (size_t)norm_len[t]);
            /* norm weights are bf16 in the checkpoint, widened to f32 by the loader */
            uint16_t *tmp = malloc(sizeof(uint16_t) * (size_t)norm_len[t]);
            oref_synth_bf16(seed, tid(src, 4 + t), (size_t)norm_len[t], norm_sigma, 1, tmp);
            for (int i = 0; i < norm_len[t]; i++) m->norms[t][l][i] = oref_bf16_to_f32(tmp[i]);
            free(tmp);
        }
        m->router[l] = malloc(sizeof(uint16_t) * (size_t)c->experts * h);
        oref_synth_bf16(seed, tid(src, 8), (size_t)c->experts * h, sigma, 0, m->router[l]);
    }
    m->embed = malloc(sizeof(uint16_t) * (size_t)c->vocab * h);
    m->lm_head = malloc(sizeof(uint16_t) * (size_t)c->vocab * h);
    oref_synth_bf16(seed, 1, (size_t)c->vocab * h, 0.02f, 0, m->embed);
    oref_synth_bf16(seed, 2, (size_t)c->vocab * h, 0.02f, 0, m->lm_head);
    uint16_t *fn = malloc(sizeof(uint16_t) * (size_t)h);
    m->final_norm = malloc(sizeof(float) * (size_t)h);
    oref_synth_bf16(seed, 3, (size_t)h, norm_sigma, 1, fn);
    for (int i = 0; i < h; i++) m->final_norm[i] = oref_bf16_to_f32(fn[i]);
    free(fn);
    return m;
}

void oref_model_free(oref_model *m) {
    if (!m) return;
    for (int l = 0; l < m->cfg.layers; l++) {
        for (int t = 0; t < 4; t++) {
            free(m->w[t][l]);
            free(m->s[t][l]);
            free(m->norms[t][l]);
        }
        free(m->router[l]);
    }
    for (int t = 0; t < 4; t++) { free(m->w[t]); free(m->s[t]); free(m->norms[t]); }
    free(m->router);
    free(m->embed);
    free(m->lm_head);
    free(m->final_norm);
    free(m);
}

const void *oref_model_tensor(const oref_model *m, int layer, int kind, const void **scale_out) {
    if (scale_out) *scale_out = NULL;
    if (kind >= 0 && kind < 4) {
        if (scale_out) *scale_out = m->s[kind][layer];
        return m->w[kind][layer];
    }
    if (kind == 4) return m->router[layer];
    if (kind >= 5 && kind <= 8) return m->norms[kind - 5][layer];
    return NULL;
}
const uint16_t *oref_model_embed(const oref_model *m) { return m->embed; }
const uint16_t *oref_model_lm_head(const oref_model *m) { return m->lm_head; }
const float *oref_model_final_norm(const oref_model *m) { return m->final_norm; }

/* ================================================================= engine step */

struct oref_engine {
    const oref_model *m;
    oref_dattn *kv;
    int pos, refined, threads;
    float *x;
    uint32_t *route_ids;
    float *route_w, *route_margin;
};

oref_engine *oref_engine_new(const oref_model *m, int max_pos, int refined_router, int threads) {
    oref_engine *e = calloc(1, sizeof(*e));
    e->m = m;
    e->kv = oref_dattn_alloc(m->cfg.layers, max_pos, m->cfg.rope_theta);
    for (int l = 0; l < m->cfg.layers; l++) oref_dattn_set_norms(e->kv, l, m->norms[2][l], m->norms[3][l]);
    e->refined = refined_router;
    e->threads = threads > 0 ? threads : 1;
    e->x = calloc((size_t)m->cfg.hidden, sizeof(float));
    e->route_ids = calloc((size_t)m->cfg.layers * m->cfg.top_k, sizeof(uint32_t));
    e->route_w = calloc((size_t)m->cfg.layers * m->cfg.top_k, sizeof(float));
    e->route_margin = calloc((size_t)m->cfg.layers, sizeof(float));
    return e;
}

void oref_engine_free(oref_engine *e) {
    if (!e) return;
    oref_dattn_free(e->kv);
    free(e->x); free(e->route_ids); free(e->route_w); free(e->route_margin);
    free(e);
}

int oref_engine_pos(const oref_engine *e) { return e->pos; }

/* Benchmark support (no reference counterpart): the next step runs at position pos over the
 * cache rows 0..pos-1 as they stand (written with oref_dattn_write_rows through oref_engine_kv). */
int oref_engine_seek(oref_engine *e, int pos) {
    if (pos < 0 || pos >= e->kv->max_pos) return -1;
    e->pos = pos;
    return 0;
}
oref_dattn *oref_engine_kv(oref_engine *e) { return e->kv; }

/* qwen3_moe_omega.rs:4096-4345 on the arms the decode graph runs: FP8 q|k|v and o, the fused
 * decode attention (bf16 KV), the device router (RMSNorm, logits, top-k), FP8 grouped gate|up,
 * host SwiGLU, FP8 grouped down with a row per slot, combine in slot order, residual adds,
 * final RMSNorm. The embedding row is bf16 widened (qwen3_moe_omega.rs:1108-1115). */
int oref_engine_step(oref_engine *e, uint32_t token, float *hidden_out) {
    const oref_model *m = e->m;
    const oref_config *c = &m->cfg;
    int h = c->hidden, hd = c->head_dim, qd = c->q_heads * hd;
    int qkv_n = (c->q_heads + 2 * c->kv_heads) * hd;
    int i = c->inter, K = c->top_k;
    if (e->pos >= e->kv->max_pos) return -1;
    if (c->q_heads != DA_QH || c->kv_heads != DA_KVH || hd != DA_HD) return -2;
    size_t t = token % (uint32_t)c->vocab;
    float *x = e->x;
    for (int j = 0; j < h; j++) x[j] = oref_bf16_to_f32(m->embed[t * h + j]);
    float *xn = malloc(sizeof(float) * (size_t)h);
    float *qkv = malloc(sizeof(float) * (size_t)qkv_n);
    float *att = malloc(sizeof(float) * (size_t)qd);
    float *proj = malloc(sizeof(float) * (size_t)h);
    float *post = malloc(sizeof(float) * (size_t)h);
    float *logits = malloc(sizeof(float) * (size_t)c->experts);
    float *moe = malloc(sizeof(float) * (size_t)h);
    float *gu = malloc(sizeof(float) * (size_t)K * 2 * i);
    float *act = malloc(sizeof(float) * (size_t)K * i);
    float *dn = malloc(sizeof(float) * (size_t)K * h);
    uint32_t zero = 0;
    for (int l = 0; l < c->layers; l++) {
        const float *in_norm = m->norms[g_mutant == 1 ? 1 : 0][l];
        const float *post_norm = m->norms[g_mutant == 1 ? 0 : 1][l];
        oref_rmsnorm(x, in_norm, h, c->eps, xn);
        fp8_grouped_impl(m->w[0][l], m->s[0][l], 1, qkv_n, h, 1, &zero, xn, 1, qkv, e->threads);
        oref_dattn_attend(e->kv, l, e->pos, qkv, c->eps, 1.0f, att);
        fp8_grouped_impl(m->w[1][l], m->s[1][l], 1, h, qd, 1, &zero, att, 1, proj, e->threads);
        for (int j = 0; j < h; j++) x[j] += proj[j];
        uint32_t *ids = e->route_ids + (size_t)l * K;
        float *wts = e->route_w + (size_t)l * K;
        int rc = oref_route(m->router[l], post_norm, c->experts, h, K, x, c->eps, e->refined,
                            ids, wts, post, logits);
        if (rc != 0) { e->pos = -1; return -3; }
        /* margin between the K-th and (K+1)-th logits */
        {
            float kth = logits[ids[K - 1]], best_out = -INFINITY;
            for (int ex = 0; ex < c->experts; ex++) {
                int chosen = 0;
                for (int s = 0; s < K; s++) chosen |= ids[s] == (uint32_t)ex;
                if (!chosen && logits[ex] > best_out) best_out = logits[ex];
            }
            e->route_margin[l] = kth - best_out;
        }
        fp8_grouped_impl(m->w[2][l], m->s[2][l], c->experts, 2 * i, h, K, ids, post, 1, gu, e->threads);
        for (int s = 0; s < K; s++) oref_swiglu(gu + (size_t)s * 2 * i, i, act + (size_t)s * i);
        fp8_grouped_impl(m->w[3][l], m->s[3][l], c->experts, h, i, K, ids, act, K, dn, e->threads);
        for (int j = 0; j < h; j++) moe[j] = 0.0f;
        for (int s = 0; s < K; s++)
            for (int j = 0; j < h; j++) moe[j] += wts[s] * dn[(size_t)s * h + j];
        for (int j = 0; j < h; j++) x[j] += moe[j];
    }
    oref_rmsnorm(x, m->final_norm, h, c->eps, hidden_out);
    e->pos++;
    free(xn); free(qkv); free(att); free(proj); free(post); free(logits); free(moe);
    free(gu); free(act); free(dn);
    return 0;
}

void oref_engine_logits(oref_engine *e, const float *hidden, float *logits) {
    bf16_gemv_impl(e->m->lm_head, e->m->cfg.vocab, e->m->cfg.hidden, hidden, logits, e->threads);
}

void oref_engine_last_routes(const oref_engine *e, uint32_t *ids, float *weights, float *margins) {
    size_t n = (size_t)e->m->cfg.layers * e->m->cfg.top_k;
    if (ids) memcpy(ids, e->route_ids, n * sizeof(uint32_t));
    if (weights) memcpy(weights, e->route_w, n * sizeof(float));
    if (margins) memcpy(margins, e->route_margin, (size_t)e->m->cfg.layers * sizeof(float));
}

void oref_engine_last_x(const oref_engine *e, float *x) {
    memcpy(x, e->x, sizeof(float) * (size_t)e->m->cfg.hidden);
}
