/*
 * vspec_abi.h -- layout-compatible declarations of the reference types that the
 * ROCm backend entry receives across its boundary.
 *
 * A reference build passes these structs by pointer (VspecKernelContext*,
 * VspecKVCache*) and by value (VspecBackend), so their layouts must match the
 * reference field for field.  Each block uses the reference header's include
 * guard: if the reference header was included first, its definition is used and
 * this one is skipped (they are identical in layout).
 *
 *   VspecBackend               include/vspec/kernel/backend.h:6-10
 *   VspecExecConfig, Context   include/vspec/kernel/context.h:8-21
 *   VspecQuantType, QuantMeta  include/vspec/quant/quant.h:12-26
 *   VspecSpecialQuantFormat    include/vspec/quant/formats/special_quant.h:8-11
 *   VspecKVCache               include/vspec/attention/kv_cache.h:11-30
 */
#ifndef VSPEC_ROCM_ABI_H
#define VSPEC_ROCM_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef VSPEC_QUANT_FORMATS_SPECIAL_QUANT_H
#define VSPEC_QUANT_FORMATS_SPECIAL_QUANT_H
typedef enum VspecSpecialQuantFormat {
    VSPEC_SPECIAL_QUANT_NONE = 0,
    VSPEC_SPECIAL_QUANT_Q4_K = 1
} VspecSpecialQuantFormat;
#endif

#ifndef VSPEC_QUANT_QUANT_H
#define VSPEC_QUANT_QUANT_H
typedef enum VspecQuantType {
    VSPEC_QUANT_NONE = 0,
    VSPEC_QUANT_INT2 = 2,
    VSPEC_QUANT_INT3 = 3,
    VSPEC_QUANT_INT4 = 4
} VspecQuantType;

typedef struct VspecQuantMeta {
    unsigned int schema_version;
    VspecQuantType type;
    const float* scales;
    size_t scale_count;
    VspecSpecialQuantFormat special_format;
    const void* special_data;
} VspecQuantMeta;
#endif

#ifndef VSPEC_KERNEL_CONTEXT_H
#define VSPEC_KERNEL_CONTEXT_H
typedef struct VspecExecConfig {
    size_t m;
    size_t n;
    size_t k;
    size_t flags; /* unused by the reference; bit 0 selects the paged descriptor below */
} VspecExecConfig;

typedef struct VspecKernelContext {
    void* input;
    void* weight;
    void* output;
    VspecQuantMeta qmeta;
    VspecExecConfig config;
} VspecKernelContext;
#endif

#ifndef VSPEC_KERNEL_BACKEND_H
#define VSPEC_KERNEL_BACKEND_H
typedef struct VspecBackend {
    const char* name;
    void (*launch_linear)(VspecKernelContext* ctx);
    void (*launch_attention)(VspecKernelContext* ctx);
} VspecBackend;
#endif

#ifndef VSPEC_ATTENTION_KV_CACHE_H
#define VSPEC_ATTENTION_KV_CACHE_H
/* Contiguous [max_tokens][num_heads][head_dim] fp32 cache, optionally with the
 * reference's int3 per-(token, head) codec and an fp32 mirror. */
typedef struct VspecKVCache {
    float* key;
    float* value;
    size_t max_tokens;
    size_t num_heads;
    size_t head_dim;
    size_t current_tokens;

    int int3_compressed;
    uint8_t* key_int3;
    uint8_t* value_int3;
    float* key_scales;
    float* value_scales;
    size_t block_size;
    size_t blocks_per_head;
    size_t packed_head_bytes;
    float* scratch_key_head;
    float* scratch_value_head;
    int owns_int3_buffers;
} VspecKVCache;
#endif

#ifdef __cplusplus
}
#endif

#endif
