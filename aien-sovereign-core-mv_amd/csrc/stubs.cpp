// The base-ABI entries of crates/aien-omega-gpu/abi/omega_gpu.manifest that sit outside the
// FP8 decode step (the bf16 dense matmul family, the elementwise kernels, the dense f32 GQA
// attention). They exist so the archive defines every manifest
// symbol (crates/aien-abi-conformance/src/build.rs:261-300 links against the full list); each
// answers BAD_ARGS with an explanation, touches no device and allocates nothing.
#include <cstring>

#include "runtime.hpp"

using namespace omega;

namespace {
const char *kOutside =
    "not part of the MI355X decode-step library (dense bf16 / elementwise / f32 attention paths "
    "are outside its scope)";
int refuse(Family f) {
    set_error(f, "%s", kOutside);
    return OMEGA_GPU_BAD_ARGS;
}
uint32_t g_cta_budget = OMEGA_GPU_MATMUL_MAX_CTAS;
}  // namespace

extern "C" {

int omega_gpu_matmul_bf16(uint32_t, uint32_t, uint32_t, const uint16_t *, const uint16_t *, float *,
                          OmegaGpuMatmulInfo *) {
    return refuse(F_MATMUL);
}
int omega_gpu_matmul_f32(uint32_t, uint32_t, uint32_t, const float *, const float *, float *,
                         OmegaGpuMatmulInfo *) {
    return refuse(F_MATMUL);
}
const char *omega_gpu_matmul_rc_name(int rc) { return rc_name(rc); }
void omega_gpu_matmul_cache_clear(void) {}
int omega_gpu_tensor_upload_bf16(uint32_t, uint32_t, const uint16_t *, OmegaGpuTensor **out) {
    if (out) *out = nullptr;
    return refuse(F_MATMUL);
}
int omega_gpu_tensor_upload_f32(uint32_t, uint32_t, const float *, OmegaGpuTensor **out) {
    if (out) *out = nullptr;
    return refuse(F_MATMUL);
}
void omega_gpu_tensor_free(OmegaGpuTensor *) {}
void omega_gpu_tensor_shape(const OmegaGpuTensor *, uint32_t *k, uint32_t *n) {
    if (k) *k = 0;
    if (n) *n = 0;
}
int omega_gpu_matmul_resident_bf16(uint32_t, const uint16_t *, const OmegaGpuTensor *, float *,
                                   OmegaGpuMatmulInfo *) {
    return refuse(F_MATMUL);
}
int omega_gpu_matmul_resident_f32(uint32_t, const float *, const OmegaGpuTensor *, float *,
                                  OmegaGpuMatmulInfo *) {
    return refuse(F_MATMUL);
}
const char *omega_gpu_matmul_last_error(void) { return last_error(F_MATMUL); }
int omega_gpu_matmul_is_blocked(void) { return 0; }
void omega_gpu_device_close(void) {}
void omega_gpu_matmul_set_cta_budget(uint32_t ctas) {
    g_cta_budget = ctas == 0 ? OMEGA_GPU_MATMUL_MAX_CTAS : ctas;
}
uint32_t omega_gpu_matmul_cta_budget(void) { return g_cta_budget; }
int omega_gpu_matmul_prepare(uint32_t, uint32_t, uint32_t) { return refuse(F_MATMUL); }

int omega_gpu_rmsnorm_f32(uint32_t, uint32_t, const float *, const float *, float, float *,
                          OmegaGpuEwInfo *) {
    return refuse(F_MATMUL);
}
int omega_gpu_rope_f32(uint32_t, uint32_t, const float *, const float *, const float *, float *,
                       OmegaGpuEwInfo *) {
    return refuse(F_MATMUL);
}
int omega_gpu_swiglu_f32(uint32_t, const float *, const float *, float *, OmegaGpuEwInfo *) {
    return refuse(F_MATMUL);
}
const char *omega_gpu_elementwise_rc_name(int rc) { return rc == -5 ? "UNWRITTEN" : rc_name(rc); }

int omega_gpu_gqa_attention_f32(const float *, const float *, const float *, uint32_t, uint32_t,
                                uint32_t, uint32_t, float *, OmegaGpuAttnInfo *) {
    return refuse(F_ATTN);
}
int omega_gpu_gqa_attention_rows_f32(const float *, const float *, const float *, uint32_t,
                                     uint32_t, uint32_t, uint32_t, uint32_t, float *,
                                     OmegaGpuAttnInfo *) {
    return refuse(F_ATTN);
}

}  // extern "C"
