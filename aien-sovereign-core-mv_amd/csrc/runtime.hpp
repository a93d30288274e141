// Internal runtime of libomega_gpu: one HIP stream per process, the error strings of every ABI
// family, pinned staging buffers and a device scratch area for the standalone entry points, and
// the object layouts shared by the entry points and the decode graph.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdarg>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <tuple>
#include <type_traits>

#include "omega_gpu.h"

namespace omega {

enum Family { F_FP8 = 0, F_GEMM, F_ROUTER, F_DATTN, F_BF16, F_SESSION, F_ATTN, F_MATMUL, F_COUNT };

void set_error(Family f, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error(Family f);
const char *last_error(Family f);
const char *rc_name(int rc);

// One lock for every entry point: handles are single-threaded by contract, global state (the
// stream, staging, workspaces, tuning knobs) is shared.
std::recursive_mutex &big_lock();

struct Ctx {
    int device = -1;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    char arch[64] = {0};
    int cus = 0;
    // pinned host staging (grows)
    void *pin = nullptr;
    size_t pin_bytes = 0;
    // device scratch (grows; never used by a captured graph)
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
};

// Initialises on first use (device = current device). Returns nullptr and sets the family's
// error when HIP is unavailable.
Ctx *ctx(Family f);
// Grow helpers; return false (error set) on allocation failure.
bool ensure_pinned(Family f, Ctx *c, size_t bytes);
bool ensure_scratch(Family f, Ctx *c, size_t bytes);
// Every allocation the library makes goes through these, so the allocation counters
// (omega_gpu_session_alloc_stats: allocations, bytes, failures, frees since the process started)
// cover all of them. A null pointer is not freed and not counted.
hipError_t dev_malloc(void **p, size_t bytes);
hipError_t host_malloc(void **p, size_t bytes, unsigned flags);
hipError_t dev_free(void *p);
hipError_t host_free(void *p);
template <typename T>
hipError_t dev_malloc(T **p, size_t bytes) {
    return dev_malloc(reinterpret_cast<void **>(p), bytes);
}
template <typename T>
hipError_t host_malloc(T **p, size_t bytes, unsigned flags) {
    return host_malloc(reinterpret_cast<void **>(p), bytes, flags);
}
// An allocation that a call makes on its own (not at create / upload time: the tiled weight
// twins a tensor gets on its first batched use) while the serving reservation is sealed: refused,
// counted as a stale refusal, the family's error set. Returns true when refused.
bool seal_refuses(Family f, const char *what, size_t bytes);

// The serving reservation (omega_gpu_reserve_serving / _seal / _release): while sealed, the grow
// helpers above and the calls' own allocations (seal_refuses) refuse to allocate (counted as
// stale refusals).
struct ServingState {
    bool reserved = false, sealed = false;
    OmegaGpuServingBounds bounds{};
};
ServingState &serving();
OmegaGpuAllocStats &alloc_counters();

// HIP call check: on failure sets the family error and returns CHIP_FAIL from the caller.
#define OMEGA_HIP(fam, call)                                                                    \
    do {                                                                                        \
        hipError_t e_ = (call);                                                                 \
        if (e_ != hipSuccess) {                                                                 \
            ::omega::set_error((fam), "%s: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, \
                               __LINE__);                                                       \
            return OMEGA_GPU_CHIP_FAIL;                                                         \
        }                                                                                       \
    } while (0)

inline uint64_t now_ns() {
    return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

// Per-launch GPU timestamps (the decode graph's stamp mode): when armed, the next launch made
// through OMEGA_LAUNCH has its start and end recorded by the dispatch itself
// (hipExtLaunchKernel), which is what a kernel-trace profiler reports as its duration.
struct LaunchStamp {
    hipEvent_t start = nullptr, stop = nullptr;
};
LaunchStamp &launch_stamp();  // per thread

// Graph building without stream capture: while a recorder is set on the thread, a launch made
// through OMEGA_LAUNCH becomes a kernel node of `graph` that depends on the previous one (a
// chain), and nothing runs. The node copies the argument values when it is added. Only kernel
// launches may happen while recording (the launchers the graphs use make no other stream call).
struct GraphRecorder {
    hipGraph_t graph = nullptr;
    hipGraphNode_t last = nullptr;
    hipError_t err = hipSuccess;
    uint32_t nodes = 0;
};
GraphRecorder *&graph_recorder();  // per thread; null when not recording
// Launches enqueued on st now are recorded into a graph (this library's recorder or a caller's
// stream capture) and may be replayed: no launch argument may then carry a per-call value.
bool stream_recording(hipStream_t st);

template <typename... P, typename... A>
void record_kernel(void (*kern)(P...), dim3 grid, dim3 block, unsigned shm, A &&...args) {
    GraphRecorder *r = graph_recorder();
    static_assert(sizeof...(P) == sizeof...(A), "one value per kernel parameter");
    std::tuple<std::decay_t<P>...> vals(std::forward<A>(args)...);
    void *params[sizeof...(P) ? sizeof...(P) : 1];
    std::apply([&](auto &...v) {
        size_t i = 0;
        ((params[i++] = (void *)&v), ...);
    }, vals);
    hipKernelNodeParams kp{};
    kp.func = (void *)kern;
    kp.gridDim = grid;
    kp.blockDim = block;
    kp.sharedMemBytes = shm;
    kp.kernelParams = params;
    kp.extra = nullptr;
    hipGraphNode_t node = nullptr;
    const hipError_t e =
        hipGraphAddKernelNode(&node, r->graph, r->last ? &r->last : nullptr, r->last ? 1 : 0, &kp);
    if (e != hipSuccess) {
        if (r->err == hipSuccess) r->err = e;
        return;
    }
    r->last = node;
    ++r->nodes;
}

// Builds `*exec` from the launches `enqueue()` makes (an int-returning callable: 0 or an ABI
// return code), as a chain of kernel nodes. On failure sets the family error and destroys what
// it made; *graph receives the graph the exec was instantiated from (the caller owns both).
template <typename F>
int build_graph(Family fam, const char *what, hipGraph_t *graph, hipGraphExec_t *exec, F &&enqueue) {
    *graph = nullptr;
    *exec = nullptr;
    hipError_t e = hipGraphCreate(graph, 0);
    if (e != hipSuccess) {
        set_error(fam, "%s: hipGraphCreate: %s", what, hipGetErrorString(e));
        return OMEGA_GPU_CODEGEN_FAIL;
    }
    GraphRecorder rec;
    rec.graph = *graph;
    graph_recorder() = &rec;
    const int rc = enqueue();
    graph_recorder() = nullptr;
    if (rc || rec.err != hipSuccess) {
        (void)hipGraphDestroy(*graph);
        *graph = nullptr;
        if (rc) return rc;
        set_error(fam, "%s: hipGraphAddKernelNode: %s", what, hipGetErrorString(rec.err));
        return OMEGA_GPU_CODEGEN_FAIL;
    }
    e = hipGraphInstantiate(exec, *graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(*graph);
        *graph = nullptr;
        *exec = nullptr;
        set_error(fam, "%s: instantiate: %s", what, hipGetErrorString(e));
        return OMEGA_GPU_CODEGEN_FAIL;
    }
    return OMEGA_GPU_OK;
}

// While recording: an event-record node after the chain's last node (the graph's own timeline).
inline hipError_t record_event_node(hipEvent_t ev) {
    GraphRecorder *r = graph_recorder();
    hipGraphNode_t node = nullptr;
    const hipError_t e = hipGraphAddEventRecordNode(&node, r->graph, r->last ? &r->last : nullptr,
                                                    r->last ? 1 : 0, ev);
    if (e == hipSuccess) r->last = node;
    else if (r->err == hipSuccess) r->err = e;
    return e;
}

#define OMEGA_LAUNCH(kern, grid, block, shm, st, ...)                                            \
    do {                                                                                         \
        ::omega::LaunchStamp &ls_ = ::omega::launch_stamp();                                     \
        if (::omega::graph_recorder()) {                                                         \
            ::omega::record_kernel(kern, grid, block, shm, __VA_ARGS__);                        \
        } else if (ls_.start) {                                                                  \
            hipExtLaunchKernelGGL(kern, grid, block, shm, st, ls_.start, ls_.stop, 0, __VA_ARGS__); \
            ls_.start = ls_.stop = nullptr;                                                      \
        } else {                                                                                 \
            hipLaunchKernelGGL(kern, grid, block, shm, st, __VA_ARGS__);                         \
        }                                                                                        \
    } while (0)

// elapsed of the last ev0 -> ev1 pair, ns
uint64_t event_ns(Ctx *c);
void fill_chip(char *target_chip, uint32_t *sm_arch, Ctx *c);

// ------------------------------------------------------------------ shared tunables / mutants
struct Knobs {
    int fp8_mutant = 0;
    int fp8_no_fold = 0;
    int fp8_sealed = 0;
    uint32_t fp8_cta_budget = 0;
    int gemm_mutant = 0;
    int moe_mutant = 0;
    int router_mutant = 0;
    int dattn_mutant = 0;
    uint32_t dattn_per_split = 0;
    uint32_t dattn_depth = 0;
    int bf16_mutant = 0;
    uint32_t spin_us = 0;
};
Knobs &knobs();

}  // namespace omega

// ---------------------------------------------------------------------------- object layouts
// Device layout of an FP8 tensor: row-major e4m3 bytes [experts][n][k] (a wavefront streams
// whole rows), scales f32 [experts][n/128][k/128].
// The matrix-core kernels of the batched paths read a tiled twin of the same bytes (built once on
// the device, on first batched use): block (expert, 16-row tile rt, 128-column block kb) is 2 KiB
// at ((expert * n/16 + rt) * k/128 + kb) * 2048, and inside it byte (row r, column c) sits at
// (c / 64) * 1024 + ((c % 64) / 16 * 16 + r) * 16 + c % 16 — the FP8 MFMA operand order, so each
// operand load instruction of a wavefront reads 1 KiB contiguous.
struct OmegaGpuFp8Tensor {
    uint32_t experts = 0, n = 0, k = 0;
    uint8_t *w = nullptr;
    float *s = nullptr;
    uint8_t *wt = nullptr;  // tiled twin (batched matrix-core paths), or null until first needed
};

namespace omega {
// builds t's tiled twin when it has none (synchronises the library stream; not during capture)
int fp8_ensure_tiled(Family f, OmegaGpuFp8Tensor *t);
}  // namespace omega
struct OmegaGpuBf16Tensor;
namespace omega {
// the same for a bf16 tensor (n a multiple of 16, k of 32)
int bf16_ensure_tiled(Family f, OmegaGpuBf16Tensor *t);
}  // namespace omega

// Device layout of a bf16 tensor: row-major [n][k] (n_pad == n).
// The batched lm_head reads a tiled twin (built on first batched use): block (16-row tile rt,
// 32-column block kb) is 1 KiB at (rt * k/32 + kb) * 512 elements, and inside it element
// (row r, column c) sits at ((c / 8) * 16 + r) * 8 + c % 8 — the bf16 MFMA operand order, each
// operand load instruction of a wavefront 1 KiB contiguous.
struct OmegaGpuBf16Tensor {
    uint32_t n = 0, k = 0, n_pad = 0;
    uint16_t *w = nullptr;
    uint16_t *wt = nullptr;  // tiled twin, or null until first needed
};
