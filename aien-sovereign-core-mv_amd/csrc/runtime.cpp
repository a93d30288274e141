// Internal runtime of libomega_gpu (see runtime.hpp).
#include "runtime.hpp"

#include <cstdio>
#include <cstdlib>

namespace omega {

namespace {
char g_err[F_COUNT][512];
bool g_has_err[F_COUNT];
Ctx g_ctx;
bool g_ctx_ready = false;
Knobs g_knobs;
}  // namespace

std::recursive_mutex &big_lock() {
    static std::recursive_mutex m;
    return m;
}

Knobs &knobs() { return g_knobs; }

void set_error(Family f, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err[f], sizeof(g_err[f]), fmt, ap);
    va_end(ap);
    g_has_err[f] = true;
}

void clear_error(Family f) { g_has_err[f] = false; }

const char *last_error(Family f) { return g_has_err[f] ? g_err[f] : nullptr; }

const char *rc_name(int rc) {
    switch (rc) {
    case 0: return "OK";
    case -1: return "BAD_ARGS";
    case -2: return "TOO_LARGE";
    case -3: return "CODEGEN_FAIL";
    case -4: return "CHIP_FAIL";
    case -5: return "PARITY_FAIL";
    default: return "?";
    }
}

Ctx *ctx(Family f) {
    if (g_ctx_ready) return &g_ctx;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        set_error(f, "no HIP device: %s", hipGetErrorString(e));
        return nullptr;
    }
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) {
        set_error(f, "hipGetDeviceProperties: %s", hipGetErrorString(e));
        return nullptr;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_error(f, "this library is built for gfx950 (MI355X); device 0 is %s",
                  prop.gcnArchName);
        return nullptr;
    }
    Ctx c;
    c.device = dev;
    c.cus = prop.multiProcessorCount;
    snprintf(c.arch, sizeof(c.arch), "%s", prop.gcnArchName);
    // default priority stream (never a priority stream)
    if ((e = hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking)) != hipSuccess ||
        (e = hipEventCreate(&c.ev0)) != hipSuccess || (e = hipEventCreate(&c.ev1)) != hipSuccess) {
        set_error(f, "stream/event create: %s", hipGetErrorString(e));
        return nullptr;
    }
    g_ctx = c;
    g_ctx_ready = true;
    return &g_ctx;
}

ServingState &serving() {
    static ServingState s;
    return s;
}

OmegaGpuAllocStats &alloc_counters() {
    static OmegaGpuAllocStats s{};
    return s;
}

static bool sealed_refusal(Family f, const char *what, size_t bytes, size_t held) {
    if (!serving().sealed) return false;
    ++alloc_counters().stale_refusals;
    set_error(f, "serving reservation exceeded: %s of %zu bytes requested after the seal (%zu held)", what,
              bytes, held);
    return true;
}

bool seal_refuses(Family f, const char *what, size_t bytes) { return sealed_refusal(f, what, bytes, 0); }

static hipError_t counted(hipError_t e, size_t bytes) {
    if (e == hipSuccess) {
        ++alloc_counters().allocs;
        alloc_counters().alloc_bytes += bytes;
    } else {
        ++alloc_counters().alloc_failures;
    }
    return e;
}

hipError_t dev_malloc(void **p, size_t bytes) { return counted(hipMalloc(p, bytes), bytes); }

hipError_t host_malloc(void **p, size_t bytes, unsigned flags) {
    return counted(hipHostMalloc(p, bytes, flags), bytes);
}

hipError_t dev_free(void *p) {
    if (!p) return hipSuccess;
    ++alloc_counters().frees;
    return hipFree(p);
}

hipError_t host_free(void *p) {
    if (!p) return hipSuccess;
    ++alloc_counters().frees;
    return hipHostFree(p);
}

bool ensure_pinned(Family f, Ctx *c, size_t bytes) {
    if (c->pin_bytes >= bytes) return true;
    if (sealed_refusal(f, "pinned staging", bytes, c->pin_bytes)) return false;
    if (c->pin) {
        (void)hipStreamSynchronize(c->stream);
        (void)host_free(c->pin);
    }
    c->pin = nullptr;
    c->pin_bytes = 0;
    size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
    hipError_t e = host_malloc(&c->pin, want, hipHostMallocDefault);
    if (e != hipSuccess) {
        set_error(f, "pinned staging of %zu bytes: %s", want, hipGetErrorString(e));
        return false;
    }
    c->pin_bytes = want;
    return true;
}

bool ensure_scratch(Family f, Ctx *c, size_t bytes) {
    if (c->scratch_bytes >= bytes) return true;
    if (sealed_refusal(f, "device scratch", bytes, c->scratch_bytes)) return false;
    if (c->scratch) {
        (void)hipStreamSynchronize(c->stream);
        (void)dev_free(c->scratch);
    }
    c->scratch = nullptr;
    c->scratch_bytes = 0;
    size_t want = bytes < (4u << 20) ? (4u << 20) : bytes;
    hipError_t e = dev_malloc(&c->scratch, want);
    if (e != hipSuccess) {
        set_error(f, "device scratch of %zu bytes: %s", want, hipGetErrorString(e));
        return false;
    }
    c->scratch_bytes = want;
    return true;
}

LaunchStamp &launch_stamp() {
    static thread_local LaunchStamp s;
    return s;
}

GraphRecorder *&graph_recorder() {
    static thread_local GraphRecorder *r = nullptr;
    return r;
}

bool stream_recording(hipStream_t st) {
    if (graph_recorder()) return true;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone;
}

uint64_t event_ns(Ctx *c) {
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, c->ev0, c->ev1) != hipSuccess) return 0;
    return (uint64_t)((double)ms * 1e6);
}

void fill_chip(char *target_chip, uint32_t *sm_arch, Ctx *c) {
    if (target_chip) snprintf(target_chip, 64, "MI355X %s", c ? c->arch : "gfx950");
    if (sm_arch) *sm_arch = 950;
}

}  // namespace omega

extern "C" {

void *omega_gpu_stream(void) {
    std::lock_guard<std::recursive_mutex> g(omega::big_lock());
    omega::Ctx *c = omega::ctx(omega::F_SESSION);
    return c ? (void *)c->stream : nullptr;
}

int omega_gpu_sync(void) {
    std::lock_guard<std::recursive_mutex> g(omega::big_lock());
    omega::Ctx *c = omega::ctx(omega::F_SESSION);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    OMEGA_HIP(omega::F_SESSION, hipStreamSynchronize(c->stream));
    return OMEGA_GPU_OK;
}

const char *omega_gpu_session_last_error(void) { return omega::last_error(omega::F_SESSION); }

int omega_gpu_session_set_spin_us(uint32_t us) {
    // omega's ceiling (OMEGA_GPU_SESSION_MAX_SPIN_US) is one second; above it the setting is
    // unchanged and -1 returned (crates/aien-omega-gpu/src/ffi.rs:190-195)
    if (us > 1000000u) return -1;
    omega::knobs().spin_us = us;
    return 0;
}

uint32_t omega_gpu_session_spin_us(void) { return omega::knobs().spin_us; }

}  // extern "C"
