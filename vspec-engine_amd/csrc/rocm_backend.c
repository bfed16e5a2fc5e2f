/*
 * rocm_backend.c -- the ROCm entry of the reference's kernel registry.
 *
 * Replaces the stub rocm_backend_stub.c:3-21.  A reference build selects it with
 * backend_preference = rocm (hw_performance_manager.c:280-284) or in auto order
 * after CUDA (:300-308); vspec_attention_forward (runtime.c:641-647) then lands in
 * rocm_launch_attention.
 */
#include <stdlib.h>
#include <string.h>

#include "vspec_rocm.h"

void vspec_rocm_set_error_(const char* msg);
int vspec_rocm_attention_cache_host(const float* q, const VspecKVCache* cache, int32_t numerics,
                                    float* out);

/* The reference decides its attention numerics from the environment on every
 * call (three_bit_runtime_modules.c:18-24, :60-66); the contiguous path honours
 * the same switch so that it agrees with the CPU backend under one environment. */
static int rocm_numerics_from_env(void) {
    const char* fb = getenv("VSPEC_FUSED_BITS");
    if (fb && fb[0] == '3' && fb[1] == '\0') {
        return VSPEC_NUMERICS_3BIT;
    }
    const char* m = getenv("VSPEC_3BIT_RUNTIME_MODULE");
    if (m && (m[0] == '1' || m[0] == 'y' || m[0] == 'Y' || m[0] == 't' || m[0] == 'T')) {
        return VSPEC_NUMERICS_3BIT;
    }
    return VSPEC_NUMERICS_PLAIN;
}

static void rocm_launch_linear(VspecKernelContext* ctx) {
    (void)ctx;
    vspec_rocm_set_error_("launch_linear: weight GEMMs are not provided by the ROCm paged-KV backend");
}

static void rocm_launch_attention(VspecKernelContext* ctx) {
    if (!ctx || !ctx->weight) {
        vspec_rocm_set_error_("launch_attention: null context or weight");
        return;
    }
    if (ctx->config.flags & VSPEC_KCTX_FLAG_PAGED) {
        (void)vspec_rocm_paged_decode_attention((const VspecPagedAttnDesc*)ctx->weight);
        return;
    }
    if (!ctx->input || !ctx->output) {
        vspec_rocm_set_error_("launch_attention: null input or output");
        return;
    }
    const VspecKVCache* cache = (const VspecKVCache*)ctx->weight;
    if (cache->current_tokens == 0) {
        return; /* attention_ref.c:12-14 leaves the output untouched */
    }
    /* fp32 rows, or int3 codes and scales when a compressed cache has no fp32 mirror */
    (void)vspec_rocm_attention_cache_host((const float*)ctx->input, cache, rocm_numerics_from_env(),
                                          (float*)ctx->output);
}

int vspec_rocm_backend_available(void) { return vspec_rocm_device_count() > 0 ? 1 : 0; }

VspecBackend vspec_make_rocm_backend(void) {
    VspecBackend backend;
    backend.name = "rocm-gfx950";
    backend.launch_linear = rocm_launch_linear;
    backend.launch_attention = rocm_launch_attention;
    return backend;
}
