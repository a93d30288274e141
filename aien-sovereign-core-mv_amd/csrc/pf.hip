// Whole-prompt prefill kernels for gfx950 (omega_gpu_pf_*): the activation quantiser, the grouped
// W8A8 GEMM over a tile table, the router logits in the packed layout, the MoE weighted combine,
// and the session memory the prefill driver allocates.
//
// Boundary: crates/aien-omega-pf/src/lib.rs:384-456 (the extern "C" blocks) with the semantics of
// its host mirrors: build_tiles (:122-160, the tile table), router_logits_ref (:505-517, the
// sequential f32 router sum from -0.0 over the packed layout of pack_router, :466-478),
// moe_combine_ref (:519-539, the slot-order combine from +0.0) and the quantiser of
// crates/aien-inference-abi/src/qwen3_moe_omega_prefill/fake_quant.rs:31-104 (power-of-two block
// scale, e4m3 round-to-nearest-even saturating to 448), whose golden table is pq_golden.txt.
// The driver that calls them is qwen3_moe_omega_prefill.rs:483-760 (WholePromptPrefill::run).
//
// Every entry is synchronous: it returns after the chip finished, with the chip nanoseconds of
// its launches (HIP events on the library stream) in *ns, also added to the module's counters.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include <pthread.h>

#include "device.hpp"
#include "kernels.hpp"
#include "mfma.hpp"
#include "runtime.hpp"

namespace omega {

// One tile-table entry, byte for byte the reference's Tile (aien-omega-pf/src/lib.rs:83-93).
typedef OmegaGpuPfTile PfTile;

constexpr uint32_t kPfBm = 64;  // activation rows per tile
constexpr uint32_t kPfLayoutPlain = 0, kPfLayoutSwiglu = 2;

// ------------------------------------------------------------------ quantiser
// f32 -> e4m3 code, round to nearest even, saturating to +-448, on the f32 bits (no dependence on
// the float mode registers): below 2^-6 the codes are the multiples of 2^-9, above it the three
// mantissa bits round on the 20 dropped ones.
__device__ __forceinline__ uint32_t e4m3_rne_sat(float f) {
    const uint32_t b = __float_as_uint(f), s = (b >> 24) & 0x80u, a = b & 0x7fffffffu;
    if (a > 0x43e00000u) return s | 0x7eu;  // above 448 (and infinities)
    if (a < 0x3c800000u) return s | (uint32_t)rintf(__uint_as_float(a) * 512.0f);
    uint32_t e = (a >> 23) - 120u, m = (a >> 20) & 7u;
    const uint32_t rem = a & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (m & 1u))) {
        if (++m == 8u) {
            m = 0;
            ++e;
        }
    }
    const uint32_t code = (e << 3) | m;
    return s | (code > 0x7eu ? 0x7eu : code);
}

struct PfQuantArgs {
    uint32_t k = 0, rows = 0, bf16_in = 0;
    const void *x = nullptr;
    uint8_t *q = nullptr;  // [rows][k]
    float *s = nullptr;    // [rows][k / 128]
};

// one wavefront per (row, 128-block): lane l holds values 2 l, 2 l + 1
__global__ __launch_bounds__(256) void k_pf_quant(const PfQuantArgs a) {
    const uint32_t blocks = a.k / 128;
    const uint32_t item = blockIdx.x * 4 + (threadIdx.x >> 6), lane = lane_id();
    if (item >= a.rows * blocks) return;
    const uint32_t row = item / blocks, b = item % blocks;
    const size_t at = (size_t)row * a.k + 128 * b + 2 * lane;
    float v0, v1;
    if (a.bf16_in) {
        const uint32_t w = *as_global_u32(static_cast<const uint16_t *>(a.x) + at);
        v0 = __uint_as_float(w << 16);
        v1 = __uint_as_float(w & 0xffff0000u);
    } else {
        const u32x2 w = *as_global_u32x2(static_cast<const float *>(a.x) + at);
        v0 = __uint_as_float(w.x);
        v1 = __uint_as_float(w.y);
    }
    float m = fmaxf(fabsf(v0), fabsf(v1));
    m = row16_max(m);
    m = fmaxf(fmaxf(readlane_f32(m, 0), readlane_f32(m, 16)), fmaxf(readlane_f32(m, 32), readlane_f32(m, 48)));
    m = fmaxf(m, 7.888609052210118e-31f);  // 2^-100
    // scale 2^(E - 8), or 2^(E - 7) when the mantissa is above 1.75 (E the exponent of m)
    const uint32_t mb = __float_as_uint(m), e = mb >> 23, c = ((mb & 0x7fffffu) + 0x1fffffu) >> 23;
    const float scale = __uint_as_float((e + c - 8u) << 23), inv = __uint_as_float((262u - e - c) << 23);
    const uint32_t q = e4m3_rne_sat(v0 * inv) | (e4m3_rne_sat(v1 * inv) << 8);
    *reinterpret_cast<uint16_t *>(a.q + at) = (uint16_t)q;
    if (lane == 0) a.s[(size_t)row * blocks + b] = scale;
}

// ------------------------------------------------------------------ grouped W8A8 GEMM
// Workgroup = (tile of up to 64 activation rows of one expert, column span); wavefront w takes
// two 16-row A tiles of the expert's row-major e4m3 weights: PLAIN, output columns
// 128 x + 32 w .. +32; SWIGLU, gate rows j0 .. j0 + 16 and up rows I + j0 .. with j0 = 64 x + 16 w
// (their act columns). The tile's activation rows (gathered through the row index) are staged per
// 128-column k-block in LDS (rows padded to 144 bytes: the 16 rows a read instruction touches sit
// on distinct banks) and shared by the four wavefronts. Per k-block, the e4m3 products run on the
// matrix cores with the activation block scale as the B operand's E8M0 scale (a power of two, so
// the products stay exact) and the f32 block sum is multiplied by the weight block scale into the
// accumulator. Two k-block sets take turns on one straight path (the loads of one in flight while
// the other is staged and multiplied); a set past the last k-block reloads the last one and
// contributes with weight scale 0.
struct PfGemmArgs {
    uint32_t n = 0, k = 0, layout = 0;
    const PfTile *tiles = nullptr;
    const uint32_t *rowidx = nullptr;  // nullptr: output row r reads activation row r
    const uint8_t *xq = nullptr;       // [rows][k] e4m3
    const float *xs = nullptr;         // [rows][k / 128]
    void *y = nullptr;                 // PLAIN f32 [rows][n]; SWIGLU bf16 [rows][n / 2]
};

constexpr uint32_t kPfRow = 144;  // staged bytes per activation row

struct PfSet {
    u32x4 a[2][2];  // A tiles: lane (g, n): row n, bytes 16 g .. +16 and 64 + 16 g .. +16
    u32x4 b[2];     // staged activation bytes: thread t: row t / 4, bytes 32 (t % 4) .. +32
    float bs;       // thread t < 64: the block scale of row t
};

template <int LAYOUT>
__global__ __launch_bounds__(256) void k_pf_qgemm(const PfGemmArgs a) {
    __shared__ __align__(16) uint8_t xb[2][kPfBm * kPfRow];
    __shared__ float xsb[2][kPfBm];
    const uint32_t tid = threadIdx.x, lane = lane_id(), w = tid >> 6, g = lane >> 4, n = lane & 15;
    const PfTile *tp = a.tiles + blockIdx.y;
    const cu32 *tw = as_const_u32(tp);
    const uint64_t w_va = (uint64_t)tw[0] | ((uint64_t)tw[1] << 32);
    const uint64_t s_va = (uint64_t)tw[2] | ((uint64_t)tw[3] << 32);
    const uint32_t row0 = tw[4], cnt = tw[5];
    const uint32_t KB = a.k / 128;
    uint32_t ra[2];
    if (LAYOUT == kPfLayoutSwiglu) {
        const uint32_t j0 = 64 * blockIdx.x + 16 * w;
        ra[0] = j0;
        ra[1] = a.n / 2 + j0;
    } else {
        ra[0] = 128 * blockIdx.x + 32 * w;
        ra[1] = ra[0] + 16;
    }
    const uint8_t *wt = reinterpret_cast<const uint8_t *>(w_va);
    const float *ws = reinterpret_cast<const float *>(s_va);
    const uint8_t *wa0 = wt + (size_t)(ra[0] + n) * a.k + 16 * g;
    const uint8_t *wa1 = wt + (size_t)(ra[1] + n) * a.k + 16 * g;
    const cu32 *ws0 = as_const_u32(ws + (size_t)(ra[0] >> 7) * KB);
    const cu32 *ws1 = as_const_u32(ws + (size_t)(ra[1] >> 7) * KB);
    // the activation row this thread stages (rows past cnt are read, never stored)
    const uint32_t srow_i = row0 + (tid >> 2);
    const uint32_t src = a.rowidx ? *as_global_u32(a.rowidx + srow_i) : srow_i;
    const uint8_t *xrow = a.xq + (size_t)src * a.k + 32 * (tid & 3);
    const uint32_t brow_i = row0 + (tid & 63);
    const uint32_t bsrc = a.rowidx ? *as_global_u32(a.rowidx + brow_i) : brow_i;
    const float *xsrow = a.xs + (size_t)bsrc * KB;

    auto load = [&](PfSet &S, uint32_t kb) {
        S.a[0][0] = __builtin_nontemporal_load(as_global(wa0 + 128 * kb));
        S.a[0][1] = __builtin_nontemporal_load(as_global(wa0 + 128 * kb + 64));
        S.a[1][0] = __builtin_nontemporal_load(as_global(wa1 + 128 * kb));
        S.a[1][1] = __builtin_nontemporal_load(as_global(wa1 + 128 * kb + 64));
        S.b[0] = *as_global(xrow + 128 * kb);
        S.b[1] = *as_global(xrow + 128 * kb + 16);
        S.bs = *as_global_f32(xsrow + kb);
    };
    f32x4 tot[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) tot[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    // stage set S (k-block kb, weight scale factor live: 1 or 0) into buffer u, then multiply
    auto step = [&](const PfSet &S, uint32_t kb, float live, int u) {
        uint8_t *xbu = xb[u];
        *reinterpret_cast<u32x4 *>(xbu + (tid >> 2) * kPfRow + 32 * (tid & 3)) = S.b[0];
        *reinterpret_cast<u32x4 *>(xbu + (tid >> 2) * kPfRow + 32 * (tid & 3) + 16) = S.b[1];
        if (tid < 64) xsb[u][tid] = S.bs;
        __syncthreads();
        const float w0 = __uint_as_float(ws0[kb]) * live, w1 = __uint_as_float(ws1[kb]) * live;
        const i32x8 A0 = {(int)S.a[0][0].x, (int)S.a[0][0].y, (int)S.a[0][0].z, (int)S.a[0][0].w,
                          (int)S.a[0][1].x, (int)S.a[0][1].y, (int)S.a[0][1].z, (int)S.a[0][1].w};
        const i32x8 A1 = {(int)S.a[1][0].x, (int)S.a[1][0].y, (int)S.a[1][0].z, (int)S.a[1][0].w,
                          (int)S.a[1][1].x, (int)S.a[1][1].y, (int)S.a[1][1].z, (int)S.a[1][1].w};
#pragma unroll
        for (int bt = 0; bt < 4; ++bt) {
            const uint8_t *r = xbu + (16 * bt + n) * kPfRow + 16 * g;
            const u32x4 b0 = *reinterpret_cast<const u32x4 *>(r);
            const u32x4 b1 = *reinterpret_cast<const u32x4 *>(r + 64);
            const i32x8 B = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
            const int sb = e8m0_of(xsb[u][16 * bt + n]);
            const f32x4 c0 = mfma_fp8_sb(A0, B, f32x4{0.f, 0.f, 0.f, 0.f}, sb);
            const f32x4 c1 = mfma_fp8_sb(A1, B, f32x4{0.f, 0.f, 0.f, 0.f}, sb);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                tot[0][bt][i] = fmaf(c0[i], w0, tot[0][bt][i]);
                tot[1][bt][i] = fmaf(c1[i], w1, tot[1][bt][i]);
            }
        }
    };
    PfSet P, Q;
    const uint32_t last = KB - 1;
    load(P, 0);
    load(Q, min(1u, last));
    for (uint32_t kb = 0; kb < KB; kb += 2) {
        step(P, kb, 1.0f, 0);
        load(P, min(kb + 2, last));
        step(Q, min(kb + 1, last), kb + 1 < KB ? 1.0f : 0.0f, 1);
        load(Q, min(kb + 3, last));
    }
    // epilogue: accumulator lane (g, n) of (A tile i, B tile bt) holds rows 4 g .. 4 g + 3 of A
    // tile i for activation row 16 bt + n
#pragma unroll
    for (int bt = 0; bt < 4; ++bt) {
        const uint32_t r = 16 * bt + n;
        if (r >= cnt) continue;
        if (LAYOUT == kPfLayoutSwiglu) {
            const uint32_t I = a.n / 2;
            uint16_t o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float gg = tot[0][bt][i], uu = tot[1][bt][i];
                o[i] = bf16_rne(gg / (1.0f + expf(-gg)) * uu);
            }
            uint16_t *yr = static_cast<uint16_t *>(a.y) + (size_t)(row0 + r) * I + ra[0] + 4 * g;
            *reinterpret_cast<u32x2 *>(yr) = u32x2{(uint32_t)o[0] | ((uint32_t)o[1] << 16),
                                                   (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
        } else {
            float *yr = static_cast<float *>(a.y) + (size_t)(row0 + r) * a.n;
            *reinterpret_cast<f32x4 *>(yr + ra[0] + 4 * g) = tot[0][bt];
            *reinterpret_cast<f32x4 *>(yr + ra[1] + 4 * g) = tot[1][bt];
        }
    }
}

// ------------------------------------------------------------------ router logits
// logits[r][ex] = (((-0.0 + w[ex][0] x[r][0]) + w[ex][1] x[r][1]) + ...): each product rounded to
// f32, then added in index order (no fused multiply-add), the reference's sequential f32 sum. The
// sum cannot be split along k, so the parallelism is (row, expert): one lane per expert, R rows
// per lane as R independent chains. The packed layout wq[g][ex][q] = w[ex][4 g + q] gives a
// wavefront of 64 experts one contiguous KiB per group of 4 columns; the R rows of x are staged
// through LDS in passes of kPfRouterKc columns and read as broadcasts, and the weight groups are
// loaded kPfRouterNg at a time in two register sets so the next set is in flight while one is
// summed. Rows come in tiles of kPfRouterRows (the buffers hold whole tiles): 16, the reference
// engine's rows per CTA that the reference's own tests expect of router_rows()
// (aien-omega-pf/src/lib.rs:1300); a launch takes 4, 2 or 1 rows per lane of such tiles.
constexpr uint32_t kPfRouterRows = 16;
constexpr uint32_t kPfRouterKc = 1024;
constexpr uint32_t kPfRouterNg = 4;

struct PfRouterArgs {
    uint32_t k = 0, e = 0, rows = 0;
    const float *x = nullptr, *wq = nullptr;
    float *logits = nullptr;
};

template <int R>
__global__ __launch_bounds__(256) void k_pf_router(const PfRouterArgs a) {
#pragma clang fp contract(off)  // a multiply then an add, never one fused rounding
    constexpr uint32_t NG = kPfRouterNg, KQ = kPfRouterKc / 4;
    __shared__ f32x4 xs[R][KQ];
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    const uint32_t ex = blockIdx.x * nt + tid;
    const uint32_t exl = ex < a.e ? ex : a.e - 1;  // lanes past the last expert load its weights
    const uint32_t r0 = blockIdx.y * R;
    const size_t gs = (size_t)a.e * 4;
    const float *wp = a.wq + (size_t)exl * 4;
    float acc[R];
#pragma unroll
    for (int j = 0; j < R; ++j) acc[j] = -0.0f;
    auto sum_group = [&](const f32x4 w, uint32_t q) {
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const f32x4 xv = xs[j][q];
            acc[j] = acc[j] + w.x * xv.x;
            acc[j] = acc[j] + w.y * xv.y;
            acc[j] = acc[j] + w.z * xv.z;
            acc[j] = acc[j] + w.w * xv.w;
        }
    };
    const uint32_t ng = a.k / 4;
    for (uint32_t c0 = 0; c0 < ng; c0 += KQ) {
        const uint32_t cn = ng - c0 < KQ ? ng - c0 : KQ;  // groups in this pass
        __syncthreads();                                  // the previous pass is read
        for (uint32_t i = tid; i < R * cn; i += nt) {
            const uint32_t j = i / cn, q = i - j * cn;
            xs[j][q] = *as_global_f32x4(a.x + (size_t)(r0 + j) * a.k + 4 * (size_t)(c0 + q));
        }
        __syncthreads();
        const float *wc = wp + (size_t)c0 * gs;
        auto load = [&](f32x4 (&w)[NG], uint32_t q) {
#pragma unroll
            for (uint32_t i = 0; i < NG; ++i) w[i] = *as_global_f32x4(wc + (size_t)(q + i) * gs);
        };
        auto sum_set = [&](const f32x4 (&w)[NG], uint32_t q) {
#pragma unroll
            for (uint32_t i = 0; i < NG; ++i) sum_group(w[i], q + i);
        };
        uint32_t q = 0;
        if (cn >= 2 * NG) {
            f32x4 A[NG], B[NG];
            load(A, 0);
            for (; q + 2 * NG <= cn; q += 2 * NG) {
                load(B, q + NG);
                sum_set(A, q);
                const uint32_t qa = q + 2 * NG <= cn - NG ? q + 2 * NG : cn - NG;  // stays in the pass
                load(A, qa);
                sum_set(B, q + NG);
            }
            if (q + NG <= cn) {  // A holds the set at q
                sum_set(A, q);
                q += NG;
            }
        }
        for (; q < cn; ++q) sum_group(*as_global_f32x4(wc + (size_t)q * gs), q);
    }
    if (ex < a.e) {
#pragma unroll
        for (int j = 0; j < R; ++j) a.logits[(size_t)(r0 + j) * a.e + ex] = acc[j];
    }
}

// ------------------------------------------------------------------ MoE combine
// out[r][c] = sum over slots in order, from +0.0, of wt[r][slot] * down[inv[r][slot]][c] (each
// product rounded, then added). One thread per (row, column).
struct PfCombineArgs {
    uint32_t h = 0, top_k = 0, rows = 0;
    const float *down = nullptr;
    const uint32_t *inv = nullptr;
    const float *wt = nullptr;
    float *out = nullptr;
};

__global__ __launch_bounds__(256) void k_pf_combine(const PfCombineArgs a) {
#pragma clang fp contract(off)  // a multiply then an add, never one fused rounding
    const uint32_t r = blockIdx.y, c = blockIdx.x * 256 + threadIdx.x;
    if (c >= a.h) return;
    float acc = 0.0f;
    for (uint32_t s = 0; s < a.top_k; ++s) {
        const uint32_t src = *as_global_u32(a.inv + (size_t)r * a.top_k + s);
        const float w = *as_global_f32(a.wt + (size_t)r * a.top_k + s);
        acc = acc + w * *as_global_f32(a.down + (size_t)src * a.h + c);
    }
    a.out[(size_t)r * a.h + c] = acc;
}

// ------------------------------------------------------------------ residual add + RMSNorm (extension)
// Per row: x += add (when given, in place), then out = x * scale * w with scale = (1 / sqrt(mean
// of squares + eps)) rounded to f32 and the squares summed in f64 (tensor.rs:94-110), so the
// driver's residual stays on the device between the GEMMs.
struct PfNormArgs {
    uint32_t k = 0;
    float *x = nullptr;
    const float *add = nullptr, *w = nullptr;
    float eps = 1e-6f;
    float *out = nullptr;
};

__global__ __launch_bounds__(256) void k_pf_resid_norm(const PfNormArgs a) {
#pragma clang fp contract(off)  // x + add and x * scale * w each rounded as written
    __shared__ double red[4];
    const uint32_t r = blockIdx.x, t = threadIdx.x, lane = lane_id(), wid = t >> 6;
    float *xr = a.x + (size_t)r * a.k;
    const float *ar = a.add ? a.add + (size_t)r * a.k : nullptr;
    double ss = 0.0;
    for (uint32_t c = t; c < a.k; c += 256) {
        float v = xr[c];
        if (ar) {
            v = v + ar[c];
            xr[c] = v;
        }
        ss += (double)v * (double)v;
    }
    ss = wave_sum_f64(ss);
    if (lane == 0) red[wid] = ss;
    __syncthreads();
    const float scale = rms_scale((red[0] + red[1]) + (red[2] + red[3]), a.k, a.eps);
    float *orow = a.out + (size_t)r * a.k;
    for (uint32_t c = t; c < a.k; c += 256) orow[c] = xr[c] * scale * a.w[c];
}

// ------------------------------------------------------------------ host threads for per-token host work
// The MoE plan of a long prompt ranks every token on the host (MoeBatchPlan::from_logits). A few
// threads, started on first use and kept for the process, split such a loop into contiguous
// ranges; the caller takes a range too. One job at a time (the entry points hold the library
// lock). The pool is never destroyed (its threads end with the process, nothing joins them at
// exit), and a child forked from the process has none of its threads: there width() is 1 and
// the caller runs the loop alone. The fork handlers hold the pool's lock across the fork so the
// child does not inherit it taken by a worker.
class HostPool {
  public:
    static HostPool &get() {
        static HostPool *p = new HostPool();
        return *p;
    }
    uint32_t width() const { return forked_ ? 1u : (uint32_t)th_.size() + 1; }
    // fn(part) for part in 0 .. parts - 1, over the pool and the calling thread. The job lives on
    // this frame: a thread takes it under the lock and counts itself in `users`, and run() returns
    // only when every part has finished and no thread still holds the job.
    void run(uint32_t parts, const std::function<void(uint32_t)> &fn) {
        Job job{&fn, parts};
        {
            std::lock_guard<std::mutex> lk(mu_);
            cur_ = &job;
            ++gen_;
        }
        cv_.notify_all();
        work(job);
        std::unique_lock<std::mutex> lk(mu_);
        done_.wait(lk, [&] { return job.finished.load() == parts && job.users == 0; });
        cur_ = nullptr;
    }

  private:
    struct Job {
        const std::function<void(uint32_t)> *fn;
        uint32_t parts;
        std::atomic<uint32_t> next{0}, finished{0};
        uint32_t users = 0;  // guarded by mu_
    };
    HostPool() {
        const unsigned hc = std::thread::hardware_concurrency();
        const unsigned n = std::min(hc ? hc : 1u, 16u);  // a one-GPU share of the host
        pthread_atfork([] { get().mu_.lock(); }, [] { get().mu_.unlock(); },
                       [] {
                           get().forked_ = true;
                           get().mu_.unlock();
                       });
        for (unsigned i = 1; i < n; ++i) th_.emplace_back([this] { loop(); });
    }
    static void work(Job &j) {
        for (uint32_t p; (p = j.next.fetch_add(1)) < j.parts;) {
            (*j.fn)(p);
            j.finished.fetch_add(1);
        }
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            Job *j;
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return cur_ && gen_ != seen; });
                seen = gen_;
                j = cur_;
                ++j->users;
            }
            work(*j);
            {
                std::lock_guard<std::mutex> lk(mu_);
                --j->users;
            }
            done_.notify_all();
        }
    }
    std::mutex mu_;
    std::condition_variable cv_, done_;
    std::vector<std::thread> th_;
    Job *cur_ = nullptr;
    uint64_t gen_ = 0;
    bool forked_ = false;
};

// ------------------------------------------------------------------ session memory and counters
struct PfState {
    std::mutex mu;
    uint64_t chip_ns = 0, launches = 0;
    uint32_t next_index = 1;
};
PfState &pf_state() {
    static PfState s;
    return s;
}

// Times the launches of `enqueue` on the library stream; adds them to the counters.
template <class F>
int pf_timed(Family fam, uint32_t launches, uint64_t *ns, F enqueue) {
    Ctx *c = ctx(fam);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    OMEGA_HIP(fam, hipEventRecord(c->ev0, c->stream));
    OMEGA_HIP(fam, enqueue(c->stream));
    OMEGA_HIP(fam, hipEventRecord(c->ev1, c->stream));
    OMEGA_HIP(fam, hipEventSynchronize(c->ev1));
    float ms = 0.f;
    OMEGA_HIP(fam, hipEventElapsedTime(&ms, c->ev0, c->ev1));
    const uint64_t t = (uint64_t)((double)ms * 1e6);
    if (ns) *ns = t;
    std::lock_guard<std::mutex> lk(pf_state().mu);
    pf_state().chip_ns += t;
    pf_state().launches += launches;
    return OMEGA_GPU_OK;
}

}  // namespace omega

using namespace omega;

extern "C" {

const char *omega_gpu_pf_rc_name(int rc) { return rc_name(rc); }

static int pf_alloc(size_t bytes, OmegaGpuMem *out, bool host) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!out || bytes == 0) {
        set_error(F_SESSION, "pf alloc: NULL out or 0 bytes");
        return OMEGA_GPU_BAD_ARGS;
    }
    memset(out, 0, sizeof(*out));
    if (!ctx(F_SESSION)) return OMEGA_GPU_CHIP_FAIL;
    void *p = nullptr, *dp = nullptr;
    if (host) {
        // host-visible, not cached by the GPU: the CPU reads and writes it in place
        OMEGA_HIP(F_SESSION, host_malloc(&p, bytes, hipHostMallocMapped | hipHostMallocCoherent));
        hipError_t e = hipHostGetDevicePointer(&dp, p, 0);
        if (e != hipSuccess) {
            (void)host_free(p);
            set_error(F_SESSION, "pf alloc host: hipHostGetDevicePointer: %s", hipGetErrorString(e));
            return OMEGA_GPU_CHIP_FAIL;
        }
        memset(p, 0, bytes);
    } else {
        OMEGA_HIP(F_SESSION, dev_malloc(&dp, bytes));
        hipError_t e = hipMemset(dp, 0, bytes);
        if (e != hipSuccess) {
            (void)dev_free(dp);
            set_error(F_SESSION, "pf alloc dev: hipMemset: %s", hipGetErrorString(e));
            return OMEGA_GPU_CHIP_FAIL;
        }
    }
    {
        std::lock_guard<std::mutex> sl(pf_state().mu);
        out->handle_index = pf_state().next_index++;
    }
    out->handle_generation = 1;
    out->kind = host ? 1u : 0u;
    out->cpu = p;
    out->va = (uint64_t)(uintptr_t)dp;
    out->size = bytes;
    return OMEGA_GPU_OK;
}

int omega_gpu_pf_alloc_dev(size_t bytes, OmegaGpuMem *out) { return pf_alloc(bytes, out, false); }
int omega_gpu_pf_alloc_host(size_t bytes, OmegaGpuMem *out) { return pf_alloc(bytes, out, true); }

void omega_gpu_pf_free(OmegaGpuMem *m) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    if (!m || !m->va) return;
    Ctx *c = ctx(F_SESSION);
    if (c) (void)hipStreamSynchronize(c->stream);
    if (m->kind == 1) (void)host_free(m->cpu);
    else (void)dev_free((void *)(uintptr_t)m->va);
    memset(m, 0, sizeof(*m));
}

int omega_gpu_pf_copy_va(uint64_t dst_va, uint64_t src_va, size_t bytes) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!dst_va || !src_va || dst_va % 16 || src_va % 16 || bytes % 16) {
        set_error(F_SESSION, "pf copy: addresses and %zu bytes must be non-zero 16-byte multiples", bytes);
        return OMEGA_GPU_BAD_ARGS;
    }
    return pf_timed(F_SESSION, 1, nullptr, [&](hipStream_t st) {
        return hipMemcpyAsync((void *)(uintptr_t)dst_va, (const void *)(uintptr_t)src_va, bytes,
                              hipMemcpyDeviceToDevice, st);
    });
}

void omega_gpu_pf_stats(uint64_t *chip_ns, uint64_t *launches) {
    std::lock_guard<std::mutex> lk(pf_state().mu);
    if (chip_ns) *chip_ns = pf_state().chip_ns;
    if (launches) *launches = pf_state().launches;
}

void omega_gpu_pf_stats_reset(void) {
    std::lock_guard<std::mutex> lk(pf_state().mu);
    pf_state().chip_ns = 0;
    pf_state().launches = 0;
}

int omega_gpu_pf_quant(uint32_t k, uint32_t in_type, uint32_t rows, uint64_t x_va, uint64_t q_va, uint64_t s_va,
                       uint64_t *ns) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (k % 128 || k < 128 || k > 32768 || in_type > 1 || !x_va || !q_va || !s_va) {
        set_error(F_SESSION, "pf quant k=%u in_type=%u refused: k a multiple of 128 in 128..=32768, "
                  "f32 (0) or bf16 (1) input, non-NULL addresses", k, in_type);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (ns) *ns = 0;
    if (rows == 0) return OMEGA_GPU_OK;
    PfQuantArgs a;
    a.k = k;
    a.rows = rows;
    a.bf16_in = in_type;
    a.x = (const void *)(uintptr_t)x_va;
    a.q = (uint8_t *)(uintptr_t)q_va;
    a.s = (float *)(uintptr_t)s_va;
    const uint64_t waves = (uint64_t)rows * (k / 128);
    if ((waves + 3) / 4 > 0x7fffffffull) {
        set_error(F_SESSION, "pf quant: %u rows of %u too large", rows, k);
        return OMEGA_GPU_TOO_LARGE;
    }
    return pf_timed(F_SESSION, 1, ns, [&](hipStream_t st) {
        OMEGA_LAUNCH(k_pf_quant, dim3((uint32_t)((waves + 3) / 4)), dim3(256), 0, st, a);
        return hipGetLastError();
    });
}

uint32_t omega_gpu_pf_qgemm_bm(void) { return kPfBm; }

uint32_t omega_gpu_pf_qgemm_tiles_va(uint32_t experts, const uint64_t *w_va, const uint64_t *s_va,
                                     const uint32_t *counts, void *tab, uint32_t max) {
    if (!w_va || !s_va || !counts || !tab || experts == 0) return 0;
    PfTile *t = static_cast<PfTile *>(tab);
    uint32_t n = 0, row = 0;
    for (uint32_t e = 0; e < experts; ++e) {
        for (uint32_t r = 0; r < counts[e];) {
            const uint32_t c = std::min(counts[e] - r, kPfBm);
            if (n >= max) return 0;
            t[n].w_va = w_va[e];
            t[n].s_va = s_va[e];
            t[n].row0 = row + r;
            t[n].cnt = c;
            t[n].pad = 0;
            ++n;
            r += c;
        }
        row += counts[e];
    }
    return n;
}

int omega_gpu_pf_moe_plan(uint32_t tokens, uint32_t experts, uint32_t top_k, const float *logits, uint32_t *topk_ids,
                          float *topk_weights, uint32_t *counts, uint32_t *grouped_token,
                          uint32_t *assignment_to_grouped, uint32_t *grouped_to_assignment) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());  // the session's error slot
    clear_error(F_SESSION);
    if (experts == 0 || experts > 65536 || top_k == 0 || top_k > experts || top_k > 64 ||
        (uint64_t)tokens * top_k > 0xffffffffull || !logits || !topk_ids || !topk_weights || !counts ||
        !grouped_token || !assignment_to_grouped) {
        set_error(F_SESSION, "pf moe plan: experts=%u, top_k=%u (1..=min(experts, 64)), tokens=%u, non-NULL "
                  "buffers", experts, top_k, tokens);
        return OMEGA_GPU_BAD_ARGS;
    }
    // the total order of f32 (f32::total_cmp) as a signed key: negative values count down
    auto key = [](float v) {
        const int32_t b = (int32_t)__builtin_bit_cast(uint32_t, v);
        return b ^ (int32_t)((uint32_t)(b >> 31) >> 1);
    };
    // tokens t0 .. t1 - 1: top_k by (key descending, id ascending), insertion into a sorted list
    // of top_k; returns the first non-finite logit's index (token * experts + expert) or ~0
    auto rank = [&](uint32_t t0, uint32_t t1) -> uint64_t {
        for (uint32_t t = t0; t < t1; ++t) {
            const float *row = logits + (size_t)t * experts;
            uint32_t sel[64];
            int32_t sk[64];
            uint32_t n = 0;
            for (uint32_t e = 0; e < experts; ++e) {
                if (!std::isfinite(row[e])) return (uint64_t)t * experts + e;
                const int32_t k = key(row[e]);
                if (n == top_k && k <= sk[n - 1]) continue;  // a tie goes to the lower id, already held
                uint32_t i = n < top_k ? n++ : n - 1;
                while (i > 0 && sk[i - 1] < k) {
                    sk[i] = sk[i - 1];
                    sel[i] = sel[i - 1];
                    --i;
                }
                sk[i] = k;
                sel[i] = e;
            }
            const float mx = row[sel[0]];
            float prob[64], sum = 0.0f;
            for (uint32_t j = 0; j < top_k; ++j) {
                prob[j] = std::exp(row[sel[j]] - mx);
                sum += prob[j];
            }
            for (uint32_t j = 0; j < top_k; ++j) {
                topk_ids[(size_t)t * top_k + j] = sel[j];
                topk_weights[(size_t)t * top_k + j] = prob[j] / sum;
            }
        }
        return ~0ull;
    };
    // long prompts: contiguous token ranges over the host threads (the results do not depend on
    // the split); the first non-finite logit in row order is the one reported
    constexpr uint32_t kTokensPerPart = 64;
    uint64_t bad = ~0ull;
    HostPool &pool = HostPool::get();
    if (tokens >= 4 * kTokensPerPart && pool.width() > 1) {
        const uint32_t parts = std::min(pool.width() * 4, (tokens + kTokensPerPart - 1) / kTokensPerPart);
        const uint32_t per = (tokens + parts - 1) / parts;
        std::vector<uint64_t> first(parts, ~0ull);
        pool.run(parts, [&](uint32_t p) {
            const uint32_t t0 = std::min(tokens, p * per), t1 = std::min(tokens, t0 + per);
            first[p] = rank(t0, t1);
        });
        for (uint64_t f : first) bad = std::min(bad, f);
    } else {
        bad = rank(0, tokens);
    }
    if (bad != ~0ull) {
        set_error(F_SESSION, "pf moe plan: logit of token %u, expert %u is not finite", (uint32_t)(bad / experts),
                  (uint32_t)(bad % experts));
        return OMEGA_GPU_BAD_ARGS;
    }
    for (uint32_t e = 0; e < experts; ++e) counts[e] = 0;
    for (uint64_t a = 0; a < (uint64_t)tokens * top_k; ++a) ++counts[topk_ids[a]];
    // stable counting sort of the assignments by expert
    std::vector<uint32_t> cursor(experts);
    uint32_t acc = 0;
    for (uint32_t e = 0; e < experts; ++e) {
        cursor[e] = acc;
        acc += counts[e];
    }
    const uint64_t assignments = (uint64_t)tokens * top_k;
    for (uint64_t a = 0; a < assignments; ++a) {
        const uint32_t g = cursor[topk_ids[a]]++;
        assignment_to_grouped[a] = g;
        grouped_token[g] = (uint32_t)(a / top_k);
        if (grouped_to_assignment) grouped_to_assignment[g] = (uint32_t)a;
    }
    return OMEGA_GPU_OK;
}

int omega_gpu_pf_qgemm(uint32_t n, uint32_t k, uint32_t layout, uint64_t tiles_va, uint32_t ntiles,
                       uint64_t rowidx_va, uint64_t xq_va, uint64_t xs_va, uint64_t y_va, uint64_t *ns) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    const uint64_t row_bytes = layout == kPfLayoutSwiglu ? n : 4ull * n;
    if (k % 128 || k < 128 || k > 32768) {
        set_error(F_SESSION, "pf qgemm k=%u refused: multiple of 128, 128 <= k <= 32768", k);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (n == 0 || n % 128 || row_bytes * kPfBm >= (1ull << 23) || (layout != kPfLayoutPlain && layout != kPfLayoutSwiglu)) {
        set_error(F_SESSION, "pf qgemm n=%u layout=%u refused: positive multiple of 128, row bytes x 64 < 2^23, "
                  "layout PLAIN (0) or SWIGLU_NAT (2)", n, layout);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (layout == kPfLayoutSwiglu && n % 256) {
        set_error(F_SESSION, "pf qgemm SwiGLU n=%u refused: multiple of 256", n);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (ntiles > 65535) {
        set_error(F_SESSION, "pf qgemm %u tiles > 65535", ntiles);
        return OMEGA_GPU_TOO_LARGE;
    }
    if (!tiles_va || !xq_va || !xs_va || !y_va) {
        set_error(F_SESSION, "pf qgemm: null address");
        return OMEGA_GPU_BAD_ARGS;
    }
    if (ns) *ns = 0;
    if (ntiles == 0) return OMEGA_GPU_OK;
    PfGemmArgs a;
    a.n = n;
    a.k = k;
    a.layout = layout;
    a.tiles = reinterpret_cast<const PfTile *>(tiles_va);
    a.rowidx = reinterpret_cast<const uint32_t *>(rowidx_va);
    a.xq = reinterpret_cast<const uint8_t *>(xq_va);
    a.xs = reinterpret_cast<const float *>(xs_va);
    a.y = reinterpret_cast<void *>(y_va);
    return pf_timed(F_SESSION, 1, ns, [&](hipStream_t st) {
        if (layout == kPfLayoutSwiglu)
            OMEGA_LAUNCH(k_pf_qgemm<kPfLayoutSwiglu>, dim3(n / 2 / 64, ntiles), dim3(256), 0, st, a);
        else
            OMEGA_LAUNCH(k_pf_qgemm<kPfLayoutPlain>, dim3(n / 128, ntiles), dim3(256), 0, st, a);
        return hipGetLastError();
    });
}

uint32_t omega_gpu_pf_router_rows(void) { return kPfRouterRows; }

void omega_gpu_pf_router_pack(uint32_t e, uint32_t k, const float *w, float *wq) {
    if (!w || !wq || k % 4) return;
    for (uint32_t g = 0; g < k / 4; ++g)
        for (uint32_t ex = 0; ex < e; ++ex)
            for (uint32_t q = 0; q < 4; ++q) wq[((size_t)g * e + ex) * 4 + q] = w[(size_t)ex * k + 4 * g + q];
    for (uint32_t i = 0; i < 4 * e; ++i) wq[(size_t)(k / 4) * e * 4 + i] = 0.f;  // the pad group
}

int omega_gpu_pf_router_logits(uint32_t k, uint32_t e, uint32_t rows, uint64_t x_va, uint64_t wq_va,
                               uint64_t logits_va, uint64_t *ns) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!x_va || !wq_va || !logits_va || k == 0 || k % 4 || e == 0 || e > 1024 || x_va % 16 || wq_va % 16) {
        set_error(F_SESSION, "pf router logits: k=%u (a multiple of 4), e=%u (1..=1024), 16-byte aligned "
                  "non-NULL x and packed weights", k, e);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (ns) *ns = 0;
    if (rows == 0) return OMEGA_GPU_OK;
    PfRouterArgs a;
    a.k = k;
    a.e = e;
    a.rows = (rows + kPfRouterRows - 1) / kPfRouterRows * kPfRouterRows;  // whole tiles
    a.x = reinterpret_cast<const float *>(x_va);
    a.wq = reinterpret_cast<const float *>(wq_va);
    a.logits = reinterpret_cast<float *>(logits_va);
    // a workgroup spans up to 256 experts; R rows per lane when that still gives one wavefront
    // per SIMD (1024 on the chip), else fewer
    const uint32_t waves_e = (e + 63) / 64, ew = waves_e < 4 ? waves_e : 4, nt = 64 * ew;
    const uint32_t gx = (e + nt - 1) / nt;
    const uint64_t waves1 = (uint64_t)gx * ew * a.rows;
    const int r = waves1 >= 4 * 1024ull ? 4 : waves1 >= 2 * 1024ull ? 2 : 1;
    const uint32_t max_rows = 32768 * (uint32_t)r;  // grid.y stays within 32768 row groups
    const uint32_t launches = (a.rows + max_rows - 1) / max_rows;
    return pf_timed(F_SESSION, launches, ns, [&](hipStream_t st) {
        for (uint32_t r0 = 0; r0 < a.rows; r0 += max_rows) {
            PfRouterArgs b = a;
            b.rows = a.rows - r0 < max_rows ? a.rows - r0 : max_rows;
            b.x = a.x + (size_t)r0 * k;
            b.logits = a.logits + (size_t)r0 * e;
            const dim3 grid(gx, b.rows / r);
            if (r == 4)
                OMEGA_LAUNCH(k_pf_router<4>, grid, dim3(nt), 0, st, b);
            else if (r == 2)
                OMEGA_LAUNCH(k_pf_router<2>, grid, dim3(nt), 0, st, b);
            else
                OMEGA_LAUNCH(k_pf_router<1>, grid, dim3(nt), 0, st, b);
            const hipError_t err = hipGetLastError();
            if (err != hipSuccess) return err;
        }
        return hipSuccess;
    });
}

int omega_gpu_pf_moe_combine(uint32_t h, uint32_t top_k, uint32_t rows, uint64_t down_va, uint64_t inv_va,
                             uint64_t wt_va, uint64_t out_va, uint64_t *ns) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!down_va || !inv_va || !wt_va || !out_va || h == 0 || top_k == 0 || top_k > 64 || rows > 65535) {
        set_error(F_SESSION, "pf moe combine: null address, h=%u, top_k=%u (1..=64) or %u rows (<= 65535)", h,
                  top_k, rows);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (ns) *ns = 0;
    if (rows == 0) return OMEGA_GPU_OK;
    PfCombineArgs a;
    a.h = h;
    a.top_k = top_k;
    a.rows = rows;
    a.down = reinterpret_cast<const float *>(down_va);
    a.inv = reinterpret_cast<const uint32_t *>(inv_va);
    a.wt = reinterpret_cast<const float *>(wt_va);
    a.out = reinterpret_cast<float *>(out_va);
    return pf_timed(F_SESSION, 1, ns, [&](hipStream_t st) {
        OMEGA_LAUNCH(k_pf_combine, dim3((h + 255) / 256, rows), dim3(256), 0, st, a);
        return hipGetLastError();
    });
}

int omega_gpu_pf_residual_norm(uint32_t k, uint32_t rows, uint64_t x_va, uint64_t add_va, uint64_t w_va, float eps,
                               uint64_t out_va, uint64_t *ns) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (k == 0 || k > 65536 || !x_va || !w_va || !out_va || rows > 0x7fffffffu) {
        set_error(F_SESSION, "pf residual norm: k=%u (1..=65536), non-NULL x, weights and out", k);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (ns) *ns = 0;
    if (rows == 0) return OMEGA_GPU_OK;
    PfNormArgs a;
    a.k = k;
    a.x = reinterpret_cast<float *>(x_va);
    a.add = reinterpret_cast<const float *>(add_va);
    a.w = reinterpret_cast<const float *>(w_va);
    a.eps = eps;
    a.out = reinterpret_cast<float *>(out_va);
    return pf_timed(F_SESSION, 1, ns, [&](hipStream_t st) {
        OMEGA_LAUNCH(k_pf_resid_norm, dim3(rows), dim3(256), 0, st, a);
        return hipGetLastError();
    });
}

}  // extern "C"
